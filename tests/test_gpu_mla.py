"""GPU parity of the MLA decode / prefill / layer entry points against the oracle.

Full DeepSeek-R1 MLA dimensions; the oracle (oracle/ref_ops.py, torch on the
CPU with the reference's rounding points) runs on identical seeded inputs.
"""
import ctypes
import functools

import pytest
import torch

from oracle import ref_ops as R
from amla import ops, synth, torch_ops
from amla._lib import lib
from amla.config import DeepSeekConfig
from _tol import assert_bf16_ulps, assert_closer_than, assert_parity

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
R1 = DeepSeekConfig()


@functools.lru_cache(maxsize=2)
def _layer(tag):
    return synth.make_layer(R1, tag)


@functools.lru_cache(maxsize=1)
def _rope(n):
    return R.precompute_rope_freqs(R1, n)


def _to_dev(aw):
    return {k: (tuple(t.to(DEV) for t in v) if isinstance(v, tuple) else v.to(DEV)) for k, v in aw.items()}


def _run_case(tag, B, S, positions, max_seq, filled=None, layer_mode=False, max_context=None):
    """Runs oracle and GPU on the same inputs; returns (gpu_out, ref_out, gpu_cache, ref_cache)."""
    print(f"[case] {tag} B={B} S={S} positions={positions} max_seq={max_seq} layer={layer_mode}", flush=True)
    lay = _layer("mla/" + tag.split(":")[0])
    hidden = synth.make_hidden(R1, B, S, tag)
    if filled is None:
        filled = list(positions) if not isinstance(positions, int) else [positions] * B
    ckv, kpe = synth.make_kv_cache(R1, B, max_seq, filled, tag)
    tab = _rope(max_seq)
    ref_ckv, ref_kpe = ckv.clone(), kpe.clone()
    if isinstance(positions, int):
        if layer_mode:
            want = R.transformer_layer_attention(hidden, lay.input_layernorm, lay.attn_weights, (ref_ckv, ref_kpe),
                                                 positions, tab, R1)
        else:
            want = R.mla_attention(hidden, lay.attn_weights, (ref_ckv, ref_kpe), positions, tab, R1)
    else:
        assert not layer_mode
        want = R.mla_attention_per_sequence(hidden, lay.attn_weights, (ref_ckv, ref_kpe), positions, tab, R1)
    aw = _to_dev(lay.attn_weights)
    g_ckv, g_kpe = ckv.to(DEV), kpe.to(DEV)
    if layer_mode:
        got = ops.mla_layer(hidden.to(DEV), lay.input_layernorm.to(DEV), aw, (g_ckv, g_kpe), positions,
                            tab.to(DEV), R1, max_context=max_context)
    else:
        got = ops.mla_attention(hidden.to(DEV), aw, (g_ckv, g_kpe), positions, tab.to(DEV), R1,
                                max_context=max_context)
    torch.cuda.synchronize()
    return got.cpu(), want, (g_ckv.cpu(), g_kpe.cpu()), (ref_ckv, ref_kpe)


def _check_cache(gc, rc, rows):
    for b, (lo, hi) in enumerate(rows):
        assert_bf16_ulps(gc[0][b, lo:hi], rc[0][b, lo:hi], 2, "ckv rows")
        assert_bf16_ulps(gc[1][b, lo:hi], rc[1][b, lo:hi], 2, "kpe rows")
    # nothing else was touched
    mask = torch.ones(gc[0].shape[:2], dtype=torch.bool)
    for b, (lo, hi) in enumerate(rows):
        mask[b, lo:hi] = False
    assert torch.equal(gc[0][mask], rc[0][mask]) and torch.equal(gc[1][mask], rc[1][mask])


def _check_layer_cache(gc, rc, hidden, gamma, aw, lo, hi):
    """Cache rows written by the layer entry (input RMSNorm first).  Decode of more than one
    sequence folds that norm into the q_a|kv_a projection's K parts: it projects bf16(x * gamma)
    and scales the fp32 sums by the row's rsqrt(mean(x^2) + eps), so the normed input is never
    rounded to bf16 as in inference/ops.py:12.  The rows then agree with the oracle to the output
    tolerance (not to 2 bf16 ulps) and are about as close as the oracle (within 10%) to the
    float64 projection of the exactly normed input.  (One sequence normalises exactly:
    test_layer_mode_batch1_cache_rows.)"""
    cfg = R1
    x = hidden.double()
    xn = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + cfg.rms_norm_eps) * gamma.double()
    w = R.fp8_block_dequant(*aw["kv_a_proj_with_mqa"]).double()
    kva = xn @ w.T
    lora = cfg.kv_lora_rank
    for i, what in ((0, "ckv rows"), (1, "kpe rows")):
        got = gc[i][:, lo:hi].float()
        want = rc[i][:, lo:hi].float()
        assert_parity(got, want, f"layer {what}")
        t = kva[..., :lora] if i == 0 else kva[..., lora:]
        assert_closer_than(got, want, t, f"layer {what} vs fp64", factor=1.1)
    # nothing else was touched
    for i in (0, 1):
        mask = torch.ones(gc[i].shape[:2], dtype=torch.bool)
        mask[:, lo:hi] = False
        assert torch.equal(gc[i][mask], rc[i][mask])


def test_decode_t257(golden):
    got, want, gc, rc = _run_case("decode257", 1, 1, 256, 264)
    assert_parity(got, want, "decode B=1 T=257")
    _check_cache(gc, rc, [(256, 257)])
    # the reference's own output for these inputs (tests/golden/make_golden.py)
    tens, man = golden
    e = man["r1_decode_t257"]
    lay = synth.make_layer(R1, e["tag"])
    if synth.sha256_of(lay.attn_weights["o_proj"][0]) == e["sha256"]["o_proj"]:
        hidden = synth.make_hidden(R1, 1, 1, e["tag"])
        ckv, kpe = synth.make_kv_cache(R1, 1, e["max_seq"], e["filled"], e["tag"])
        tab = R.precompute_rope_freqs(R1, e["max_seq"]).to(DEV)
        out = ops.mla_attention(hidden.to(DEV), _to_dev(lay.attn_weights), (ckv.to(DEV), kpe.to(DEV)), 256, tab, R1)
        assert_parity(out.cpu(), tens["r1_decode_t257.out"].view(torch.bfloat16), "decode vs reference golden")


def test_prefill_s8_vs_reference_golden(golden):
    """amla_mla_prefill on the inputs of the reference's own R1 prefill of 8 tokens
    (tests/golden/make_golden.py wrote the reference's output and cache rows)."""
    from test_oracle import _rebuild
    tens, man = golden
    e = man["r1_prefill_s8"]
    print("[case] prefill S=8 vs reference golden", flush=True)
    cfg, lay, hidden, ckv, kpe = _rebuild(e)
    assert synth.sha256_of(hidden) == e["sha256"]["hidden"]
    assert synth.sha256_of(lay.attn_weights["o_proj"][0]) == e["sha256"]["o_proj"]
    tab = R.precompute_rope_freqs(cfg, e["max_seq"]).to(DEV)
    c = (ckv.to(DEV), kpe.to(DEV))
    out = ops.mla_attention(hidden.to(DEV), _to_dev(lay.attn_weights), c, e["position"], tab, cfg)
    torch.cuda.synchronize()
    assert_parity(out.cpu(), tens["r1_prefill_s8.out"].view(torch.bfloat16), "prefill S=8 vs reference golden")
    p, S = e["position"], e["S"]
    assert_bf16_ulps(c[0][:, p:p + S].cpu(), tens["r1_prefill_s8.ckv_new"].view(torch.bfloat16), 2, "ckv rows")
    assert_bf16_ulps(c[1][:, p:p + S].cpu(), tens["r1_prefill_s8.kpe_new"].view(torch.bfloat16), 2, "kpe rows")


@pytest.mark.parametrize("S,layer", [(1, False), (1, True), (40, False), (40, True)])
def test_unit_gammas(S, layer):
    """Every RMSNorm weight exactly 1 (q_a_layernorm, kv_a_layernorm and the layer's input norm):
    the gamma folded into the absorbed query, the latent and the GEMM inputs is then the identity,
    so this isolates the rest of each path."""
    tag = f"gamma1/S{S}/L{int(layer)}"
    print(f"[case] unit gammas S={S} layer={layer}", flush=True)
    lay = synth.make_layer(R1, tag, gamma_mode="ones")
    assert bool((lay.attn_weights["q_a_layernorm"].float() == 1).all())
    B, pos, max_seq = 3, 300, 344
    hidden = synth.make_hidden(R1, B, S, tag)
    ckv, kpe = synth.make_kv_cache(R1, B, max_seq, pos, tag)
    tab = _rope(max_seq)
    rc = (ckv.clone(), kpe.clone())
    if layer:
        want = R.transformer_layer_attention(hidden, lay.input_layernorm, lay.attn_weights, rc, pos, tab, R1)
    else:
        want = R.mla_attention(hidden, lay.attn_weights, rc, pos, tab, R1)
    gc = (ckv.to(DEV), kpe.to(DEV))
    if layer:
        got = ops.mla_layer(hidden.to(DEV), lay.input_layernorm.to(DEV), _to_dev(lay.attn_weights), gc, pos,
                            tab.to(DEV), R1)
    else:
        got = ops.mla_attention(hidden.to(DEV), _to_dev(lay.attn_weights), gc, pos, tab.to(DEV), R1)
    torch.cuda.synchronize()
    assert_parity(got.cpu(), want, f"unit gammas S={S} layer={layer}")
    gc = (gc[0].cpu(), gc[1].cpu())
    if layer:
        _check_layer_cache(gc, rc, hidden, lay.input_layernorm, lay.attn_weights, pos, pos + S)
    else:
        _check_cache(gc, rc, [(pos, pos + S)] * B)


def test_decode_batch_above_64_runs_in_chunks():
    """inference/ops.py:119 takes any batch: 70 sequences (a chunk of 64 and one of 6, the
    workspace sized for 64) against the oracle."""
    B, max_seq, pos = 70, 96, 80
    got, want, gc, rc = _run_case("decode70", B, 1, pos, max_seq)
    assert_parity(got, want, "decode B=70")
    _check_cache(gc, rc, [(pos, pos + 1)] * B)
    lay = _layer("mla/decode70")
    hidden = synth.make_hidden(R1, B, 1, "decode70")
    ckv, kpe = synth.make_kv_cache(R1, B, max_seq, pos, "decode70")
    a = ops._mla_operands(hidden.to(DEV), _to_dev(lay.attn_weights), (ckv.to(DEV), kpe.to(DEV)), pos,
                          _rope(max_seq).to(DEV), R1)
    args = torch_ops.fill_mla_args(out=torch.empty_like(a["hidden"]), **a)
    small = torch_ops.fill_mla_args(out=torch.empty_like(a["hidden"][:64]), **{**a, "hidden": a["hidden"][:64]})
    assert lib().amla_mla_decode_workspace_bytes(ctypes.byref(args)) == \
        lib().amla_mla_decode_workspace_bytes(ctypes.byref(small))


def test_decode_t4096():
    got, want, gc, rc = _run_case("decode4096", 1, 1, 4095, 4096)
    assert_parity(got, want, "decode B=1 T=4096")
    _check_cache(gc, rc, [(4095, 4096)])


def test_decode_batch1_context32768_256_splits():
    """One sequence at context 32768: 256 splits of 128 rows, so the combine's merge reads
    (m, l) over four rounds of 64 lanes and each of its two parts runs seven batches of rows."""
    got, want, gc, rc = _run_case("decode32k", 1, 1, 32767, 32768)
    assert_parity(got, want, "decode B=1 T=32768")
    _check_cache(gc, rc, [(32767, 32768)])


def test_decode_batch8_shared_position():
    got, want, gc, rc = _run_case("decodeb8", 8, 1, 1023, 1030)
    assert_parity(got, want, "decode B=8 T=1024")
    _check_cache(gc, rc, [(1023, 1024)] * 8)


def test_decode_ragged_positions():
    pos = [100, 777, 1500, 31, 0]
    got, want, gc, rc = _run_case("ragged", 5, 1, pos, 1600)
    assert_parity(got, want, "ragged decode")
    _check_cache(gc, rc, [(p, p + 1) for p in pos])


def test_decode_ragged_head_groups():
    """A ragged batch with few split slots (3 sequences, 75 split units): the attention runs two
    workgroups of 64 heads per slot, both reading the split plan table of the unequal tile counts."""
    pos = [1500, 90, 777]
    got, want, gc, rc = _run_case("raggedhg", 3, 1, pos, 1600)
    assert_parity(got, want, "ragged decode, head groups")
    _check_cache(gc, rc, [(p, p + 1) for p in pos])


def test_decode_batch32_ragged():
    """Batched decode at batch 32 with ragged positions (the reference's batched-decode
    workload, at contexts the oracle finishes in seconds): 17..32-row skinny GEMMs and
    eight splits per sequence."""
    g = torch.Generator().manual_seed(32)
    pos = torch.randint(0, 300, (32,), generator=g).tolist()
    got, want, gc, rc = _run_case("ragged32", 32, 1, pos, 320)
    assert_parity(got, want, "batch-32 ragged decode")
    _check_cache(gc, rc, [(p, p + 1) for p in pos])


def test_decode_split_count_does_not_matter():
    a, want, _, _ = _run_case("splits", 2, 1, 3000, 8192, max_context=3001)
    b, _, _, _ = _run_case("splits", 2, 1, 3000, 8192, max_context=8192)
    assert_parity(a, want, "splits tight")
    assert_parity(b, want, "splits loose")
    assert_parity(a, b, "split plan independence")


def test_decode_overflow_recompute():
    """A cached rope key 500x larger than the rest, in the second tile of its
    split: heads whose score jumps more than 2^64 above the split's reference
    max take the exact recomputation path of the combine kernel.  Context 4201
    is 132 tiles of 32 rows in 66 splits of two tiles; row 1510 is in tile 47,
    the second of split 23."""
    tag = "overflow"
    lay = _layer("mla/" + tag)
    pos = 4200
    hidden = synth.make_hidden(R1, 1, 1, tag)
    ckv, kpe = synth.make_kv_cache(R1, 1, 4208, pos, tag)
    kpe[0, 1510] = (kpe[0, 1510].float() * 500).to(torch.bfloat16)
    tab = _rope(4208)
    want = R.mla_attention(hidden, lay.attn_weights, (ckv.clone(), kpe.clone()), pos, tab, R1)
    got = ops.mla_attention(hidden.to(DEV), _to_dev(lay.attn_weights), (ckv.to(DEV), kpe.to(DEV)), pos, tab.to(DEV), R1)
    assert_parity(got.cpu(), want, "overflow recompute")


def test_decode_single_position_ignores_query():
    # T = 1: softmax == 1, the output cannot depend on the query path
    lay = _layer("mla/t1")
    hidden = synth.make_hidden(R1, 1, 1, "t1").to(DEV)
    tab = _rope(8).to(DEV)
    outs = []
    for mul in (1.0, 3.0):
        aw = _to_dev(lay.attn_weights)
        w, s = aw["q_b_proj"]
        aw["q_b_proj"] = (w, s * mul)
        ckv = torch.zeros(1, 8, 512, dtype=torch.bfloat16, device=DEV)
        kpe = torch.zeros(1, 8, 64, dtype=torch.bfloat16, device=DEV)
        outs.append(ops.mla_attention(hidden, aw, (ckv, kpe), 0, tab, R1).cpu())
    assert_parity(outs[0], outs[1], "T=1 independent of q")


@pytest.mark.parametrize("S", [8, 64, 300])
def test_prefill_from_empty(S):
    got, want, gc, rc = _run_case(f"prefill{S}", 1, S, 0, S + 8)
    assert_parity(got, want, f"prefill S={S}")
    _check_cache(gc, rc, [(0, S)])


def test_prefill_1024():
    got, want, gc, rc = _run_case("prefill1024", 1, 1024, 0, 1024)
    assert_parity(got, want, "prefill S=1024")
    _check_cache(gc, rc, [(0, 1024)])


def test_prefill_chunk_after_cache():
    got, want, gc, rc = _run_case("chunk", 2, 32, 100, 200)
    assert_parity(got, want, "chunked prefill B=2 S=32 at 100")
    _check_cache(gc, rc, [(100, 132)] * 2)


def test_layer_mode_decode_and_prefill():
    for tag, B, S, pos, max_seq in (("layerdec", 2, 1, 700, 704), ("layerpre", 1, 96, 0, 96)):
        got, want, gc, rc = _run_case(tag, B, S, pos, max_seq, layer_mode=True)
        assert_parity(got, want, f"layer {tag}")
        lay = _layer("mla/" + tag)
        _check_layer_cache(gc, rc, synth.make_hidden(R1, B, S, tag), lay.input_layernorm, lay.attn_weights,
                           pos, pos + S)


def test_layer_mode_batch1_cache_rows():
    """Layer-mode decode of one sequence: the streaming q_a|kv_a GEMV applies the input RMSNorm to
    its x row with the reference's rounding (inference/ops.py:10-12), so the new cache row is
    within 2 bf16 ulps of the oracle's, like the non-layer entry's."""
    for tag, pos, max_seq in (("layerb1", 256, 264), ("layerb1b", 4095, 4104)):
        got, want, gc, rc = _run_case(tag, 1, 1, pos, max_seq, layer_mode=True)
        assert_parity(got, want, f"layer {tag}")
        _check_cache(gc, rc, [(pos, pos + 1)])


def test_layer_mode_batch8_cache_rows():
    """Layer-mode decode of 2-8 sequences: the q_a|kv_a GEMV with x in LDS normalises each x row
    with the reference's rounding (inference/ops.py:10-12) and q_b's normalises q_a, so the new
    cache rows are within 2 bf16 ulps of the oracle's."""
    for tag, B, pos, max_seq in (("layerb8", 8, 300, 304), ("layerb3", 3, 1000, 1008)):
        got, want, gc, rc = _run_case(tag, B, 1, pos, max_seq, layer_mode=True)
        assert_parity(got, want, f"layer {tag}")
        _check_cache(gc, rc, [(pos, pos + 1)] * B)


def test_layer_mode_batches_above_8():
    """Layer-mode decode of 9-64 sequences: the q_a|kv_a GEMV for 9-64 rows of x projects
    bf16(x * gamma) in K parts and the finish applies each row's norm factor (the folded input
    norm of _check_layer_cache); 24 and 40 sequences take two and four 16-row column tiles."""
    for tag, B, pos, max_seq in (("layerb24", 24, 500, 504), ("layerb40", 40, 200, 208)):
        got, want, gc, rc = _run_case(tag, B, 1, pos, max_seq, layer_mode=True)
        assert_parity(got, want, f"layer {tag}")
        lay = _layer("mla/" + tag)
        _check_layer_cache(gc, rc, synth.make_hidden(R1, B, 1, tag), lay.input_layernorm, lay.attn_weights,
                           pos, pos + 1)


def test_prefill_row_equals_decode():
    """Prefill of S tokens, row S-1 == prefill of S-1 tokens followed by a decode step."""
    lay = _layer("mla/consistency")
    aw = _to_dev(lay.attn_weights)
    S = 40
    hidden = synth.make_hidden(R1, 1, S, "consistency").to(DEV)
    tab = _rope(64).to(DEV)
    c1 = (torch.zeros(1, 64, 512, dtype=torch.bfloat16, device=DEV), torch.zeros(1, 64, 64, dtype=torch.bfloat16, device=DEV))
    full = ops.mla_attention(hidden, aw, c1, 0, tab, R1)
    c2 = (torch.zeros_like(c1[0]), torch.zeros_like(c1[1]))
    ops.mla_attention(hidden[:, :S - 1].contiguous(), aw, c2, 0, tab, R1)
    last = ops.mla_attention(hidden[:, S - 1:].contiguous(), aw, c2, S - 1, tab, R1)
    assert_parity(last.cpu(), full[:, S - 1:].cpu(), "decode step vs prefill row")
    assert_bf16_ulps(c2[0].cpu(), c1[0].cpu(), 2, "cache rows")


def test_entry_points_share_one_workspace():
    """Decode, standalone split-K fp8_linear and prefill interleaved on one
    workspace: each leaves the shared split-K counters at zero for the next."""
    a, want_a, _, _ = _run_case("share", 4, 1, 2047, 2050)
    w, s = _layer("mla/share").attn_weights["o_proj"]
    x = synth.randn((3, w.shape[1]), 77).to(torch.bfloat16)
    y = ops.fp8_linear(x.to(DEV), w.to(DEV), s.to(DEV)).cpu()
    b, want_b, _, _ = _run_case("share:pre", 1, 8, 0, 16)
    c, want_c, _, _ = _run_case("share", 4, 1, 2047, 2050)
    assert_parity(a, want_a, "decode before")
    assert_parity(y, R.fp8_linear(x, w, s), "split-K linear between")
    assert_parity(b, want_b, "prefill after decode")
    assert_parity(c, want_c, "decode after prefill")


def test_bad_arguments_raise_before_launch():
    lay = _layer("mla/t1")
    aw = _to_dev(lay.attn_weights)
    tab = _rope(8).to(DEV)
    hidden = torch.zeros(1, 1, 7168, dtype=torch.bfloat16, device=DEV)
    ckv = torch.zeros(1, 8, 512, dtype=torch.bfloat16, device=DEV)
    kpe = torch.zeros(1, 8, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        ops.mla_attention(hidden, aw, (ckv, kpe), 8, tab, R1)            # beyond the cache
    with pytest.raises(TypeError):
        ops.mla_attention(hidden.float(), aw, (ckv, kpe), 0, tab, R1)    # dtype
    with pytest.raises(ValueError):
        ops.mla_attention(hidden, aw, (ckv[:, :, :256].contiguous(), kpe), 0, tab, R1)   # cache width
    bad = dict(aw)
    bad["o_proj"] = (aw["o_proj"][0][:, :8192].contiguous(), aw["o_proj"][1])
    with pytest.raises(ValueError):
        ops.mla_attention(hidden, bad, (ckv, kpe), 0, tab, R1)


def _plan_mirror(lengths, tmax, units, slots):
    """The decode split plan: the smallest split length L (in 32-row tiles) with
    sum_b ceil(N_b / L) <= units, s_b = max(1, ceil(N_b / L)) splits per sequence in
    consecutive slots; the table as the kernels store it (L, sum s_b, two spare ints,
    (first_b, s_b) pairs, the sequence of each slot), minus the spare ints."""
    tiles = [(min(t, tmax) + 31) // 32 for t in lengths]
    fits = lambda L: sum(-(-n // L) for n in tiles) <= units
    L = next(L for L in range(1, max(tiles) + 1) if fits(L))
    s = [max(1, -(-n // L)) for n in tiles]
    first = [sum(s[:b]) for b in range(len(s))]
    pairs = [v for fk in zip(first, s) for v in fk]
    slot_seq = [-1] * slots
    for b, (f, k) in enumerate(zip(first, s)):
        slot_seq[f:f + k] = [b] * k
    longest = max(max((j + 1) * n // k - j * n // k for j in range(k)) for n, k in zip(tiles, s))
    assert longest <= L
    return [L, sum(s)], pairs + slot_seq


@pytest.mark.parametrize("case", ["ragged5", "config3", "short"])
def test_split_plan_is_the_shortest_longest_split(case):
    """The split plan table that the absorb launch writes for a batch with unequal tile
    counts (the first region of the decode workspace) equals the min-max rule above; the
    attention and the combine read it, so the parity tests check that they agree.
    Batches of equal tile counts use the same rule in closed form (no table)."""
    g = torch.Generator().manual_seed(5)
    if case == "ragged5":
        lengths, max_seq = [1 + int(v) for v in torch.randint(0, 1600, (5,), generator=g)], 1600
    elif case == "config3":
        lengths, max_seq = synth.ragged_lengths(32, 1024, 16384, "config3"), 16384
    else:
        lengths, max_seq = [1, 40, 257], 264
    B = len(lengths)
    print(f"[case] split plan {case} B={B} max_seq={max_seq}", flush=True)
    aw = _to_dev(_layer("mla/plan").attn_weights)
    hidden = synth.make_hidden(R1, B, 1, "plan").to(DEV)
    ckv = torch.zeros(B, max_seq, 512, dtype=torch.bfloat16, device=DEV)
    kpe = torch.zeros(B, max_seq, 64, dtype=torch.bfloat16, device=DEV)
    pos = torch.tensor([t - 1 for t in lengths], dtype=torch.int32)
    tab = _rope(max_seq).to(DEV)
    out = torch.empty_like(hidden)
    operands = ops._mla_operands(hidden, aw, (ckv, kpe), pos.to(DEV), tab, R1)
    a = torch_ops.fill_mla_args(out=out, **operands)
    ws = torch.empty(lib().amla_mla_decode_workspace_bytes(a), dtype=torch.uint8, device=DEV)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    assert lib().amla_mla_decode(ctypes.byref(a), torch.cuda.current_stream().cuda_stream) == 0, lib().amla_last_error()
    torch.cuda.synchronize()
    ntiles = -(-max_seq // 32)
    units = min(256, B * ntiles if B * ntiles <= 64 else B * max(1, ntiles // 2))
    slots = units + B
    head, table = _plan_mirror(lengths, max_seq, units, slots)
    got = ws[:4 * (4 + 2 * B + slots)].view(torch.int32).cpu().tolist()
    assert got[:2] == head and got[4:] == table
