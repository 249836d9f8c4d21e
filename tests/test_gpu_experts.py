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


def _shared_and_router(tag):
    shared = {p: _q(*(I, D) if p != "down_proj" else (D, I), f"{tag}/shared/{p}") for p in ("gate_proj", "up_proj", "down_proj")}
    gw = synth.randn((E, D), synth.seed_of("stream", tag, "router"), 0.1).to(torch.bfloat16)
    return shared, gw


@pytest.mark.parametrize("tokens,slots", [(8, 4), (256, 4), (3, 16)])
def test_moe_block_streams_in_waves(tokens, slots):
    """More distinct experts than pool slots: moe_block streams them in waves; bit-equal to
    moe_block over the same experts resident on the device, and within the bar of the oracle."""
    print(f"[case] streamed waves tokens={tokens} slots={slots}", flush=True)
    tab = _host_table()
    shared, gw = _shared_and_router("waves")
    sh_dev = {p: (w.to(DEV), s.to(DEV)) for p, (w, s) in shared.items()}
    st = ExpertStreamer(CFG, lambda l, e: tab[(l, e)], DEV, slots=slots)
    h = synth.randn((tokens, 1, D), synth.seed_of("stream", "waves", tokens), 1.0).to(torch.bfloat16)
    hd, gd = h.to(DEV), gw.to(DEV)
    routing = ops.route(hd, gd, CFG)
    distinct = len(torch.unique(routing[0]).tolist())
    got = ops.moe_block(hd, gd, sh_dev, st, CFG, layer=1, routing=routing)
    resident = {e: {p: (w.to(DEV), s.to(DEV)) for p, (w, s) in tab[(1, e)].items()} for e in range(E)}
    ref = ops.moe_block(hd, gd, sh_dev, resident, CFG)
    torch.cuda.synchronize()
    assert st.copies >= distinct > (slots if tokens > 3 else 0)
    assert torch.equal(got, ref)
    want = F.moe_block(h, gw, shared, lambda e: {p: (w.clone(), s.clone()) for p, (w, s) in tab[(1, e)].items()}, CFG)
    assert_parity(got, want, f"streamed waves tokens={tokens}")


def test_held_views_survive_a_prefetch():
    """Views handed out by transfer_experts are not evicted by a prefetch before their consumer
    runs; the next transfer call releases them."""
    tab = _host_table()
    st = ExpertStreamer(CFG, lambda l, e: tab[(l, e)], DEV, slots=4)
    views = st.transfer_experts(0, [0, 1])
    st.prefetch(0, [2, 3])                                 # fills the two free slots
    st.prefetch(0, [4, 5])                                 # evicts 2 and 3, never the held 0 and 1
    assert (0, 0) in st.lru and (0, 1) in st.lru and (0, 2) not in st.lru and (0, 3) not in st.lru
    with pytest.raises(RuntimeError):
        st.prefetch(0, [6, 7, 8])                          # three new experts, two slots not held
    torch.cuda.synchronize()
    for e, v in zip((0, 1), views):
        assert torch.equal(v["gate_proj"][0].cpu().view(torch.uint8), tab[(0, e)]["gate_proj"][0].view(torch.uint8))
    st.transfer_experts(0, [6, 7, 8])                      # releases 0 and 1 first
    assert st.copies == 6 + 3 and (0, 0) not in st.lru


def test_moe_block_r1_decode_batch_streamed_in_waves():
    """R1 routing (256 experts, top-8, 8 tokens) on a 16-slot pool: every chosen expert's
    weights streamed from pinned host memory in waves, bit-equal to the same experts resident."""
    from amla.config import DeepSeekConfig
    R1 = DeepSeekConfig()
    d, n = R1.hidden_size, R1.moe_intermediate_size
    print("[case] R1 decode batch, 16-slot pool", flush=True)
    gw = synth.randn((R1.n_routed_experts, d), synth.seed_of("stream", "r1", "router"), 0.05, DEV).to(torch.bfloat16)
    h = synth.randn((8, 1, d), synth.seed_of("stream", "r1", "h"), 1.0, DEV).to(torch.bfloat16)
    routing = ops.route(h, gw, R1)
    chosen = torch.unique(routing[0]).tolist()
    assert len(chosen) > 16

    def expert(e, dev):
        return {p: tuple(t.to(dev) for t in synth.quantize_fp8_blocks(
            synth.randn((n, d) if p != "down_proj" else (d, n), synth.seed_of("stream", "r1", e, p), 0.02, DEV)))
            for p in ("gate_proj", "up_proj", "down_proj")}

    resident = {e: expert(e, DEV) for e in chosen}
    host = {e: {p: tuple(t.cpu().pin_memory() for t in v) for p, v in resident[e].items()} for e in chosen}
    shared = expert(-1, DEV)
    st = ExpertStreamer(R1, lambda l, e: host[e], DEV, slots=16)
    got = ops.moe_block(h, gw, shared, st, R1, layer=3, routing=routing)
    ref = ops.moe_block(h, gw, shared, resident, R1, routing=routing)
    torch.cuda.synchronize()
    assert st.copies == len(chosen)
    assert torch.equal(got, ref)


def test_store_to_streamer_to_moe_block(tmp_path):
    """Safetensors shards -> pinned ExpertStore -> ExpertStreamer (waves on a 4-slot pool, the
    store's slots refilled only after their copies) -> moe_block, against the oracle."""
    from _ckpt import write_checkpoint
    from amla.expert_store import ExpertStore
    print("[case] store -> streamer -> moe_block", flush=True)
    ref = write_checkpoint(str(tmp_path), D, I, E, 2, tag="e2e")
    store = ExpertStore(str(tmp_path), CFG, capacity_bytes=6 * ExpertStore(str(tmp_path), CFG, 1, pinned=False).slot_bytes)
    assert store.arena.is_pinned()
    st = ExpertStreamer(CFG, store, DEV, slots=4)
    shared, gw = _shared_and_router("e2e")
    sh_dev = {p: (w.to(DEV), s.to(DEV)) for p, (w, s) in shared.items()}
    for it, tokens in enumerate((8, 40, 8)):
        layer = it % 2
        h = synth.randn((tokens, 1, D), synth.seed_of("stream", "e2e", it), 1.0).to(torch.bfloat16)
        got = ops.moe_block(h.to(DEV), gw.to(DEV), sh_dev, st, CFG, layer=layer)
        torch.cuda.synchronize()
        want = F.moe_block(h, gw, shared, lambda e: {p: (w.clone(), s.clone()) for p, (w, s) in ref[(layer, e)].items()},
                           CFG)
        assert_parity(got, want, f"store->streamer->moe it={it}")
    assert store.misses > store.capacity                   # the store itself evicted and re-read
