"""amla_mla_decode_noalloc (scratch in a static per-device array) against
amla_mla_decode (caller workspace), through the C ABI: bit-equal outputs and
cache rows on two calls in a row, the second with a smaller batch and context,
and a call that needs more scratch than the array holds is refused before any
launch."""
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


def _case(tag, B, T):
    lay = synth.make_layer(R1, tag)
    aw = {k: (tuple(t.to(DEV) for t in v) if isinstance(v, tuple) else v.to(DEV)) for k, v in lay.attn_weights.items()}
    hidden = synth.make_hidden(R1, B, 1, tag).to(DEV)
    ckv = torch.randn(B, T, 512, device=DEV).to(torch.bfloat16)
    kpe = torch.randn(B, T, 64, device=DEV).to(torch.bfloat16)
    tab = R.precompute_rope_freqs(R1, T).to(DEV)
    return aw, hidden, (ckv, kpe), tab, lay.input_layernorm.to(DEV)


def _args(aw, hidden, cache, tab, T, gamma, out):
    operands = ops._mla_operands(hidden, aw, cache, T - 1, tab, R1, input_gamma=gamma, residual=hidden)
    return torch_ops.fill_mla_args(out=out, **operands), operands


def _both(aw, hidden, cache, tab, T, gamma):
    st = torch.cuda.current_stream().cuda_stream
    c_ref = (cache[0].clone(), cache[1].clone())
    out_ref = torch.empty_like(hidden)
    a, keep = _args(aw, hidden, c_ref, tab, T, gamma, out_ref)
    ws = torch.empty(lib().amla_mla_decode_workspace_bytes(a), dtype=torch.uint8, device=DEV)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    assert lib().amla_mla_decode(ctypes.byref(a), st) == 0, lib().amla_last_error()
    c_na = (cache[0].clone(), cache[1].clone())
    out_na = torch.empty_like(hidden)
    b, keep2 = _args(aw, hidden, c_na, tab, T, gamma, out_na)
    b.workspace, b.workspace_bytes = None, 0          # ignored by the no-allocation entry point
    assert lib().amla_mla_decode_noalloc(ctypes.byref(b), st) == 0, lib().amla_last_error()
    torch.cuda.synchronize()
    return out_ref, out_na, c_ref, c_na


def test_noalloc_decode_equals_workspace_decode_twice():
    for tag, B, T in (("noalloc-big", 8, 32768), ("noalloc-small", 2, 3000)):
        print(f"[case] noalloc B={B} T={T}", flush=True)
        aw, hidden, cache, tab, gamma = _case(tag, B, T)
        out_ref, out_na, c_ref, c_na = _both(aw, hidden, cache, tab, T, gamma)
        assert torch.equal(out_na, out_ref), f"B={B} T={T}"
        assert torch.equal(c_na[0], c_ref[0]) and torch.equal(c_na[1], c_ref[1])


def test_noalloc_refuses_a_call_beyond_the_array():
    print("[case] noalloc oversize (batch 64)", flush=True)
    aw, hidden, cache, tab, gamma = _case("noalloc-over", 64, 256)
    out = torch.empty_like(hidden)
    a, keep = _args(aw, hidden, cache, tab, 256, gamma, out)
    assert lib().amla_mla_decode_workspace_bytes(a) > (48 << 20)
    before = cache[0].clone()
    rc = lib().amla_mla_decode_noalloc(ctypes.byref(a), torch.cuda.current_stream().cuda_stream)
    assert rc == -2 and b"static array" in lib().amla_last_error()
    torch.cuda.synchronize()
    assert torch.equal(cache[0], before)              # nothing was launched
