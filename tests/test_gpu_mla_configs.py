"""GPU parity of MLA decode / prefill at the full sizes of the benchmark configurations.

* batched ragged decode: batch 32, contexts drawn uniform in [1024, 16384];
* decode batch 8 at context 32768 (position 32767);
* prefill of 4096 tokens from an empty cache, plus the "prefill row i ==
  decode at position i" invariant on the cache it wrote;
* the 61-layer MLA-only stack (input RMSNorm + MLA + residual per layer) at
  batch 8, context 32768, replayed from a HIP graph: every replay equal to the
  eager run, layer 0 and layer 37 against the oracle.

Each result is checked against the oracle (the reference's rounding points) with
the elementwise, normwise and RMS bars of tests/_tol.py, per head before o_proj,
and against float64 truth (the GPU may be at most 2x further from it than the
oracle is).
"""
import functools

import pytest
import torch

from oracle import ref_ops as R
from oracle import truth as TR
from amla import ops, synth
from amla.config import DeepSeekConfig
from _tol import assert_closer_than, assert_heads_parity, assert_parity

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
R1 = DeepSeekConfig()
H, V = R1.num_attention_heads, R1.v_head_dim


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _to_dev(aw):
    return {k: (tuple(t.to(DEV) for t in v) if isinstance(v, tuple) else v.to(DEV)) for k, v in aw.items()}


@functools.lru_cache(maxsize=1)
def _layer(tag):
    return synth.make_layer(R1, tag)


def _decode_case(tag, positions, max_seq):
    """GPU decode (attn_out captured) and the oracle's per-sequence parts on the same inputs."""
    B = len(positions)
    lay = _layer(tag)
    hidden = synth.make_hidden(R1, B, 1, tag)
    ckv, kpe = synth.make_kv_cache(R1, B, max_seq, list(positions), tag)
    tab = R.precompute_rope_freqs(R1, max_seq)
    g_ckv, g_kpe = ckv.to(DEV), kpe.to(DEV)
    heads = torch.empty(B, 1, H * V, dtype=torch.bfloat16, device=DEV)
    _say(f"{tag}: GPU decode B={B} max_seq={max_seq} sum(T)={sum(p + 1 for p in positions)}")
    got = ops.mla_attention(hidden.to(DEV), _to_dev(lay.attn_weights), (g_ckv, g_kpe), list(positions),
                            tab.to(DEV), R1, attn_out=heads)
    torch.cuda.synchronize()
    _say(f"{tag}: oracle")
    ref_ckv, ref_kpe = ckv.clone(), kpe.clone()
    want_h, want = R.mla_attention_per_sequence_parts(hidden, lay.attn_weights, (ref_ckv, ref_kpe), positions,
                                                      tab, R1)
    # the rows written: the new latent + rope key at each position
    gc, gk = g_ckv.cpu(), g_kpe.cpu()
    for b, p in enumerate(positions):
        assert torch.allclose(gc[b, p].float(), ref_ckv[b, p].float(), rtol=2 ** -7, atol=1e-3)
        assert torch.allclose(gk[b, p].float(), ref_kpe[b, p].float(), rtol=2 ** -7, atol=1e-3)
    return dict(lay=lay, hidden=hidden, tab=tab, cache=(ref_ckv, ref_kpe), got=got.cpu(), heads=heads.cpu(),
                want=want, want_h=want_h)


def _truth_check(c, positions, sample, what):
    idx = list(sample)
    th, tout = TR.mla_decode_absorbed_parts_f64(c["hidden"][idx], c["lay"].attn_weights, c["cache"][0][idx],
                                                c["cache"][1][idx], [positions[i] for i in idx], c["tab"], R1)
    assert_closer_than(c["heads"][idx], c["want_h"][idx], th, f"{what} heads vs fp64")
    assert_closer_than(c["got"][idx], c["want"][idx], tout, f"{what} output vs fp64")


def test_decode_batch32_ragged_contexts_1k_16k():
    lengths = synth.ragged_lengths(32, 1024, 16384, "config3")
    positions = [L - 1 for L in lengths]
    c = _decode_case("config3", positions, max(lengths))
    assert_parity(c["got"], c["want"], "batch-32 ragged decode, contexts U[1024, 16384]")
    assert_heads_parity(c["heads"], c["want_h"], H, "batch-32 ragged decode heads")
    shortest, longest = min(range(32), key=lambda b: lengths[b]), max(range(32), key=lambda b: lengths[b])
    _truth_check(c, positions, [shortest, longest, 7], "batch-32 ragged")


def test_decode_batch8_context32768():
    positions = [32767] * 8
    c = _decode_case("config4dec", positions, 32768)
    assert_parity(c["got"], c["want"], "decode B=8 T=32768")
    assert_heads_parity(c["heads"], c["want_h"], H, "decode B=8 T=32768 heads")
    _truth_check(c, positions, [0, 5], "decode B=8 T=32768")


def test_prefill_4096_and_decode_rows():
    tag, S = "config4pre", 4096
    lay = _layer(tag)
    hidden = synth.make_hidden(R1, 1, S, tag)
    tab = R.precompute_rope_freqs(R1, S)
    aw = _to_dev(lay.attn_weights)
    g_ckv = torch.zeros(1, S, 512, dtype=torch.bfloat16, device=DEV)
    g_kpe = torch.zeros(1, S, 64, dtype=torch.bfloat16, device=DEV)
    heads = torch.empty(1, S, H * V, dtype=torch.bfloat16, device=DEV)
    _say("prefill S=4096: GPU")
    got = ops.mla_attention(hidden.to(DEV), aw, (g_ckv, g_kpe), 0, tab.to(DEV), R1, attn_out=heads).cpu()
    heads = heads.cpu()
    _say("prefill S=4096: oracle")
    ckv = torch.zeros(1, S, 512, dtype=torch.bfloat16)
    kpe = torch.zeros(1, S, 64, dtype=torch.bfloat16)
    want_h, want = R.mla_attention_parts(hidden, lay.attn_weights, (ckv, kpe), 0, tab, R1)
    assert_parity(got, want, "prefill S=4096")
    assert_heads_parity(heads, want_h, H, "prefill S=4096 heads")
    assert torch.allclose(g_ckv.cpu().float(), ckv.float(), rtol=2 ** -7, atol=1e-3)
    assert torch.allclose(g_kpe.cpu().float(), kpe.float(), rtol=2 ** -7, atol=1e-3)
    rows = [0, 1, 31, 255, 1000, 2047, 3071, 4095]
    _say(f"prefill S=4096: fp64 rows {rows}")
    th, tout = TR.mla_prefill_rows_f64(hidden, lay.attn_weights, ckv, kpe, 0, rows, tab, R1)
    assert_closer_than(heads[0, rows], want_h[0, rows], th, "prefill heads vs fp64 (sampled rows)")
    assert_closer_than(got[0, rows], want[0, rows], tout, "prefill output vs fp64 (sampled rows)")
    # row i of the prefill == one decode step at position i over the cache the prefill wrote
    for i in (511, 2048, 4095):
        _say(f"prefill S=4096: decode at position {i}")
        c2 = (g_ckv.clone(), g_kpe.clone())
        step = ops.mla_attention(hidden[:, i:i + 1].contiguous().to(DEV), aw, c2, i, tab.to(DEV), R1).cpu()
        assert_parity(step, got[:, i:i + 1], f"decode at {i} vs prefill row {i}")


def _stack(layers, B, T, tag):
    stack = [synth.make_layer(R1, tag, L, device=DEV) for L in range(layers)]
    caches = []
    for L in range(layers):
        ckv = synth.randn((B, T, 512), synth.seed_of(tag, L, "ckv"), 1.0, DEV).to(torch.bfloat16)
        kpe = synth.randn((B, T, 64), synth.seed_of(tag, L, "kpe"), 1.0, DEV).to(torch.bfloat16)
        caches.append((ckv, kpe))
    return stack, caches


def test_stack61_graph_replays_equal_eager_and_oracle():
    """61 layers x (input RMSNorm -> MLA -> residual), batch 8, context 32768: one HIP
    graph replayed three times (eager work and synchronisation between replays), each
    replay bit-equal to the eager stack; layers 0 and 37 against the oracle."""
    NL, B, T, tag = 61, 8, 32768, "stack61"
    _say(f"stack: building {NL} layers on the GPU")
    stack, caches = _stack(NL, B, T, tag)
    rope = ops.precompute_rope_freqs(R1, T, DEV)
    pos = torch.full((B,), T - 1, dtype=torch.int32, device=DEV)
    x0 = synth.randn((B, 1, R1.hidden_size), synth.seed_of(tag, "hidden"), 1.0, DEV).to(torch.bfloat16)

    def run(x):
        hs = [x]
        for lay, cache in zip(stack, caches):
            hs.append(ops.mla_layer(hs[-1], lay.input_layernorm, lay.attn_weights, cache, pos, rope, R1,
                                    max_context=T))
        return hs

    _say("stack: eager")
    eager = [h.clone() for h in run(x0)]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    static_x = x0.clone()
    with torch.cuda.graph(g):
        outs = run(static_x)
    for rep in range(3):
        _say(f"stack: graph replay {rep}")
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(outs[-1], eager[-1]), f"replay {rep} differs from eager"
        assert torch.equal(outs[38], eager[38])
        # eager work between replays (allocations, a different stream-ordered launch)
        junk = ops.mla_layer(eager[5], stack[5].input_layernorm, stack[5].attn_weights, caches[5], pos, rope, R1,
                             max_context=T)
        torch.cuda.synchronize()
        assert torch.equal(junk, eager[6])
    for L, seqs in ((0, [0, 7]), (37, [2, 5])):
        _say(f"stack: oracle layer {L} sequences {seqs}")
        lay = stack[L]
        aw = {k: (tuple(t.cpu() for t in v) if isinstance(v, tuple) else v.cpu()) for k, v in lay.attn_weights.items()}
        tab = rope.cpu()
        for b in seqs:
            ckv, kpe = caches[L][0][b:b + 1].cpu(), caches[L][1][b:b + 1].cpu()
            want = R.transformer_layer_attention(eager[L][b:b + 1].cpu(), lay.input_layernorm.cpu(), aw, (ckv, kpe),
                                                 T - 1, tab, R1)
            assert_parity(eager[L + 1][b:b + 1].cpu(), want, f"stack layer {L} sequence {b}")
