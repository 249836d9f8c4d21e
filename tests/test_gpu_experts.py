"""Expert streaming (amla.experts.ExpertStreamer, the counterpart of inference/gpu_transfer.py)
against the CPU oracle: slot contents, LRU reuse, eviction, and the MoE block fed from the slots."""
from types import SimpleNamespace

import pytest
import torch

from oracle import ref_ffn as F
from amla import ops, synth
from amla.experts import ExpertStreamer
from _tol import assert_parity

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
D, I, E = 256, 256, 16
CFG = SimpleNamespace(hidden_size=D, moe_intermediate_size=I, n_routed_experts=E, n_group=4, topk_group=2,
                      num_experts_per_tok=4, norm_topk_prob=True, routed_scaling_factor=2.5)


def _q(n, k, tag):
    return synth.quantize_fp8_blocks(synth.randn((n, k), synth.seed_of("stream", tag, n, k), 0.02))


def _host_table():
    tab = {}
    for l in range(2):
        for e in range(E):
            tab[(l, e)] = {p: tuple(t.pin_memory() for t in _q(*(I, D) if p != "down_proj" else (D, I), f"{l}/{e}/{p}"))
                           for p in ("gate_proj", "up_proj", "down_proj")}
    return tab


def test_transfer_contents_and_lru():
    tab = _host_table()
    st = ExpertStreamer(CFG, lambda l, e: tab[(l, e)], DEV, slots=8)
    got = st.transfer_experts(0, torch.tensor([3, 7, 3, 1]))
    torch.cuda.synchronize()
    assert len(got) == 4 and st.copies == 3                 # expert 3 copied once
    for e, wts in zip([3, 7, 3, 1], got):
        for p in ("gate_proj", "up_proj", "down_proj"):
            assert torch.equal(wts[p][0].cpu().view(torch.uint8), tab[(0, e)][p][0].view(torch.uint8))
            assert torch.equal(wts[p][1].cpu(), tab[(0, e)][p][1])
    st.transfer_experts(0, [1, 3])
    assert st.copies == 3                                   # resident: no copy
    st.transfer_experts(1, [1, 2, 4, 5, 6, 8])               # fills the pool, evicts the oldest
    assert st.copies == 9
    again = st.transfer_experts(0, [7])                     # 7 was evicted (oldest): copied again
    torch.cuda.synchronize()
    assert st.copies == 10
    assert torch.equal(again[0]["down_proj"][0].cpu().view(torch.uint8), tab[(0, 7)]["down_proj"][0].view(torch.uint8))
    with pytest.raises(RuntimeError):
        st.transfer_experts(1, list(range(9)))              # more distinct experts than slots


def test_moe_block_from_streamed_experts():
    tab = _host_table()
    st = ExpertStreamer(CFG, lambda l, e: tab[(l, e)], DEV, slots=8)
    shared = {p: _q(*(I, D) if p != "down_proj" else (D, I), f"shared/{p}") for p in ("gate_proj", "up_proj", "down_proj")}
    sh_dev = {p: (w.to(DEV), s.to(DEV)) for p, (w, s) in shared.items()}
    gw = synth.randn((E, D), synth.seed_of("stream", "router"), 0.1).to(torch.bfloat16)
    for it in range(4):
        layer = it % 2
        print(f"[case] streamed moe it={it}", flush=True)
        h = synth.randn((2, 1, D), synth.seed_of("stream", "h", it), 1.0).to(torch.bfloat16)
        idx, _ = ops.route(h.to(DEV), gw.to(DEV), CFG)
        experts = st.experts_for(layer, idx)
        got = ops.moe_block(h.to(DEV), gw.to(DEV), sh_dev, experts, CFG)
        torch.cuda.synchronize()
        want = F.moe_block(h, gw, shared, lambda e: {p: (w.clone(), s.clone()) for p, (w, s) in tab[(layer, e)].items()}, CFG)
        assert_parity(got, want, f"streamed moe it={it}")
