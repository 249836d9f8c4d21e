"""GPU tests of the torch.ops.amla layer: the custom-op path equals a direct C-ABI
call, torch.compile(fullgraph=True) sees and runs the ops, and per-call scratch
keeps captured HIP graphs valid across later, larger calls."""
import ctypes

import pytest
import torch

from oracle import ref_ops as R
from amla import ops, synth, torch_ops
from amla._lib import check, lib
from amla.config import DeepSeekConfig
from _tol import assert_parity

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
R1 = DeepSeekConfig()


def _to_dev(aw):
    return {k: (tuple(t.to(DEV) for t in v) if isinstance(v, tuple) else v.to(DEV)) for k, v in aw.items()}


def _inputs(tag, B, S, max_seq, filled):
    lay = synth.make_layer(R1, tag)
    hidden = synth.make_hidden(R1, B, S, tag).to(DEV)
    ckv, kpe = synth.make_kv_cache(R1, B, max_seq, filled, tag)
    tab = R.precompute_rope_freqs(R1, max_seq).to(DEV)
    return lay, _to_dev(lay.attn_weights), hidden, (ckv.to(DEV), kpe.to(DEV)), tab


def test_custom_op_equals_direct_c_abi_call():
    print("[case] op vs C ABI: decode B=3 T=1500 and fp8_linear M=5", flush=True)
    lay, aw, hidden, (ckv, kpe), tab = _inputs("opabi", 3, 1, 1504, 1499)
    c1 = (ckv.clone(), kpe.clone())
    via_op = ops.mla_attention(hidden, aw, c1, 1499, tab, R1)
    # the same call straight through amla_mla_decode with a caller-owned workspace
    c2 = (ckv.clone(), kpe.clone())
    operands = ops._mla_operands(hidden, aw, c2, 1499, tab, R1)
    out = torch.empty_like(hidden)
    a = torch_ops.fill_mla_args(out=out, **operands)
    ws = torch.empty(lib().amla_mla_decode_workspace_bytes(a), dtype=torch.uint8, device=DEV)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    check(lib().amla_mla_decode(ctypes.byref(a), torch.cuda.current_stream().cuda_stream), "mla_decode")
    torch.cuda.synchronize()
    assert torch.equal(via_op, out)
    assert torch.equal(c1[0], c2[0]) and torch.equal(c1[1], c2[1])
    w, s = aw["o_proj"]
    x = torch.randn(5, w.shape[1], device=DEV).to(torch.bfloat16)
    y_op = torch.ops.amla.fp8_linear(x, w, s)
    y = torch.empty(5, w.shape[0], dtype=torch.bfloat16, device=DEV)
    need = lib().amla_fp8_linear_workspace_bytes(5, w.shape[0], w.shape[1])
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=DEV)
    check(lib().amla_fp8_linear(x.data_ptr(), 5, w.shape[1], w.shape[1], w.data_ptr(), s.data_ptr(), w.shape[0],
                                y.data_ptr(), w.shape[0], ws.data_ptr(), ws.numel(),
                                torch.cuda.current_stream().cuda_stream), "fp8_linear")
    torch.cuda.synchronize()
    assert torch.equal(y_op, y)


def test_torch_compile_fullgraph_runs_the_ops():
    print("[case] torch.compile fullgraph: decode + prefill layers", flush=True)
    lay, aw, hidden, cache, tab = _inputs("compile", 2, 1, 520, 511)
    gamma = lay.input_layernorm.to(DEV)

    def step(h, ckv, kpe):
        return ops.mla_layer(h, gamma, aw, (ckv, kpe), 511, tab, R1)

    eager_cache = (cache[0].clone(), cache[1].clone())
    want = step(hidden, *eager_cache)
    compiled = torch.compile(step, fullgraph=True, backend="aot_eager")
    c = (cache[0].clone(), cache[1].clone())
    got = compiled(hidden, *c)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    # the compiled graph performed the in-place cache store
    assert torch.equal(c[0], eager_cache[0]) and torch.equal(c[1], eager_cache[1])
    assert not torch.equal(c[0][:, 511], cache[0][:, 511])


def test_graph_replay_after_a_larger_call_matches_eager():
    """Capture a decode, run a much larger prefill and decode eagerly (their scratch comes
    from the same allocator), replay the graph: the replay equals the eager decode."""
    print("[case] graph capture B=4 T=2048, then prefill S=1024 and decode B=8 T=8192, replay", flush=True)
    lay, aw, hidden, cache, tab = _inputs("graphsafe", 4, 1, 2056, 2047)
    ref = ops.mla_attention(hidden, aw, (cache[0].clone(), cache[1].clone()), 2047, tab, R1)
    static_cache = (cache[0].clone(), cache[1].clone())
    pos = torch.full((4,), 2047, dtype=torch.int32, device=DEV)
    ops.mla_attention(hidden, aw, static_cache, pos, tab, R1, max_context=2048)   # warm-up
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ops.mla_attention(hidden, aw, static_cache, pos, tab, R1, max_context=2048)
    _, aw2, h2, c2, t2 = _inputs("graphsafe-big", 1, 1024, 1024, 0)
    h3 = synth.make_hidden(R1, 8, 1, "graphsafe-dec").to(DEV)
    c3 = (torch.randn(8, 8192, 512, device=DEV).to(torch.bfloat16), torch.randn(8, 8192, 64, device=DEV).to(torch.bfloat16))
    t3 = R.precompute_rope_freqs(R1, 8192).to(DEV)
    for rep in range(3):
        # larger eager work in between, whose scratch comes from the same allocator
        big = ops.mla_attention(h2, aw2, c2, 0, t2, R1)
        dec = ops.mla_attention(h3, aw, c3, 8191, t3, R1)
        torch.cuda.synchronize()
        del big, dec
        torch.cuda.empty_cache()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}"


def test_two_streams_do_not_share_scratch():
    """Decodes of two different inputs issued on two streams at once equal their serial results."""
    print("[case] two streams", flush=True)
    _, aw, h1, c1, tab = _inputs("streams-a", 4, 1, 4100, 4095)
    h2 = synth.make_hidden(R1, 4, 1, "streams-b").to(DEV)
    c2 = (c1[0].clone(), c1[1].clone())
    want1 = ops.mla_attention(h1, aw, (c1[0].clone(), c1[1].clone()), 4095, tab, R1)
    want2 = ops.mla_attention(h2, aw, (c2[0].clone(), c2[1].clone()), 4095, tab, R1)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s1):
        got1 = ops.mla_attention(h1, aw, c1, 4095, tab, R1)
    with torch.cuda.stream(s2):
        got2 = ops.mla_attention(h2, aw, c2, 4095, tab, R1)
    torch.cuda.synchronize()
    assert torch.equal(got1, want1) and torch.equal(got2, want2)


def test_attn_out_is_the_pre_o_proj_activation():
    """attn_out of decode and prefill, pushed through the same o_proj linear, gives the output."""
    print("[case] attn_out decode/prefill", flush=True)
    lay, aw, hidden, cache, tab = _inputs("attnout", 2, 1, 300, 299)
    heads = torch.empty(2, 1, 128 * 128, dtype=torch.bfloat16, device=DEV)
    out = ops.mla_attention(hidden, aw, cache, 299, tab, R1, attn_out=heads)
    assert torch.equal(ops.fp8_linear(heads, *aw["o_proj"]), out)
    hp = synth.make_hidden(R1, 1, 40, "attnout-p").to(DEV)
    cp = (torch.zeros(1, 64, 512, dtype=torch.bfloat16, device=DEV), torch.zeros(1, 64, 64, dtype=torch.bfloat16, device=DEV))
    hh = torch.empty(1, 40, 128 * 128, dtype=torch.bfloat16, device=DEV)
    outp = ops.mla_attention(hp, aw, cp, 0, R.precompute_rope_freqs(R1, 64).to(DEV), R1, attn_out=hh)
    assert_parity(ops.fp8_linear(hh, *aw["o_proj"]), outp, "prefill o_proj(attn_out)")
