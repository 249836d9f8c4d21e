"""amla_mla_decode_profiled (amla_mla_decode with an event recorded before each of its seven
stages and one after the last) through the C ABI: the same output and cache rows, bit for
bit, as amla_mla_decode on the same inputs, and the eight events complete in order on the
launch stream."""
import ctypes

import pytest
import torch

from oracle import ref_ops as R
from amla import ops, synth, torch_ops
from amla._lib import lib
from amla.config import DeepSeekConfig

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
R1 = DeepSeekConfig()
NEV = 8


def _call(aw, hidden, cache, tab, T, gamma, events=None, repeat=1):
    st = torch.cuda.current_stream()
    out = torch.empty_like(hidden)
    operands = ops._mla_operands(hidden, aw, cache, T - 1, tab, R1, input_gamma=gamma, residual=hidden)
    a = torch_ops.fill_mla_args(out=out, **operands)
    ws = torch.empty(lib().amla_mla_decode_workspace_bytes(a), dtype=torch.uint8, device=DEV)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    if events is None:
        rc = lib().amla_mla_decode(ctypes.byref(a), st.cuda_stream)
    elif repeat == 1:
        arr = (ctypes.c_void_p * NEV)(*[e.cuda_event for e in events])
        rc = lib().amla_mla_decode_profiled(ctypes.byref(a), st.cuda_stream, arr)
    else:
        arr = (ctypes.c_void_p * NEV)(*[e.cuda_event for e in events])
        rc = lib().amla_mla_decode_profiled_repeat(ctypes.byref(a), st.cuda_stream, arr, repeat)
    assert rc == 0, lib().amla_last_error()
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("B,T", [(8, 4096), (3, 777)])
def test_profiled_decode_equals_decode(B, T):
    print(f"[case] decode_profiled B={B} T={T}", flush=True)
    tag = f"profiled{B}"
    lay = synth.make_layer(R1, tag)
    aw = {k: (tuple(t.to(DEV) for t in v) if isinstance(v, tuple) else v.to(DEV)) for k, v in lay.attn_weights.items()}
    gamma = lay.input_layernorm.to(DEV)
    hidden = synth.make_hidden(R1, B, 1, tag).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(B * 1000 + T)
    ckv = torch.randn(B, T, 512, device=DEV, generator=g).to(torch.bfloat16)
    kpe = torch.randn(B, T, 64, device=DEV, generator=g).to(torch.bfloat16)
    tab = R.precompute_rope_freqs(R1, T).to(DEV)
    events = [torch.cuda.Event(enable_timing=True) for _ in range(NEV)]
    st = torch.cuda.current_stream()
    for e in events:                     # torch creates the hipEvent on its first record
        e.record(st)
    torch.cuda.synchronize()
    c_ref = (ckv.clone(), kpe.clone())
    c_prof = (ckv.clone(), kpe.clone())
    want = _call(aw, hidden, c_ref, tab, T, gamma)
    got = _call(aw, hidden, c_prof, tab, T, gamma, events)
    assert torch.equal(got, want)
    assert torch.equal(c_prof[0], c_ref[0]) and torch.equal(c_prof[1], c_ref[1])
    assert all(e.query() for e in events)
    stages = [events[i].elapsed_time(events[i + 1]) for i in range(NEV - 1)]
    assert all(s >= 0 for s in stages), stages
    assert stages[4] > 0, stages         # the attention stage
    assert events[0].elapsed_time(events[-1]) == pytest.approx(sum(stages), rel=1e-3, abs=1e-3)


def test_profiled_attention_repeat_keeps_the_output():
    """amla_mla_decode_profiled_repeat: the attention kernel launched 8 times back to back
    between events 4 and 5 gives the same output and cache rows, bit for bit, and that stage
    takes several times as long as one launch."""
    B, T = 4, 8192
    print(f"[case] decode_profiled_repeat B={B} T={T}", flush=True)
    tag = "profiled-rep"
    lay = synth.make_layer(R1, tag)
    aw = {k: (tuple(t.to(DEV) for t in v) if isinstance(v, tuple) else v.to(DEV)) for k, v in lay.attn_weights.items()}
    gamma = lay.input_layernorm.to(DEV)
    hidden = synth.make_hidden(R1, B, 1, tag).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(4321)
    ckv = torch.randn(B, T, 512, device=DEV, generator=g).to(torch.bfloat16)
    kpe = torch.randn(B, T, 64, device=DEV, generator=g).to(torch.bfloat16)
    tab = R.precompute_rope_freqs(R1, T).to(DEV)
    st = torch.cuda.current_stream()
    ev1 = [torch.cuda.Event(enable_timing=True) for _ in range(NEV)]
    ev8 = [torch.cuda.Event(enable_timing=True) for _ in range(NEV)]
    for e in ev1 + ev8:
        e.record(st)
    torch.cuda.synchronize()
    c1, c8 = (ckv.clone(), kpe.clone()), (ckv.clone(), kpe.clone())
    one = _call(aw, hidden, c1, tab, T, gamma, ev1, repeat=1)
    eight = _call(aw, hidden, c8, tab, T, gamma, ev8, repeat=8)
    assert torch.equal(one, eight)
    assert torch.equal(c1[0], c8[0]) and torch.equal(c1[1], c8[1])
    t1, t8 = ev1[4].elapsed_time(ev1[5]), ev8[4].elapsed_time(ev8[5])
    assert t8 > 4 * t1, (t1, t8)
