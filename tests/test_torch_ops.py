"""The torch.ops.amla custom-op layer without a GPU: registration, schemas and
FakeTensor tracing of the reference-signature shims (no kernel runs)."""
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx
from torch._subclasses.functional_tensor import dispatch_functionalize

from amla import ops, synth, torch_ops  # noqa: F401  (registers the operators)
from amla.config import DeepSeekConfig

R1 = DeepSeekConfig()


def test_operators_are_registered_with_mutation_schemas():
    for name in ("fp8_linear", "rms_norm", "apply_rope", "mla_decode", "mla_prefill"):
        assert hasattr(torch.ops.amla, name), name
    for name in ("mla_decode", "mla_prefill"):
        schema = getattr(torch.ops.amla, name).default._schema
        mutated = {a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write}
        assert mutated == {"ckv_cache", "kpe_cache", "attn_out"}, (name, mutated)
    s = torch.ops.amla.fp8_linear.default._schema
    assert not any(a.alias_info is not None and a.alias_info.is_write for a in s.arguments)


def _fake_inputs(mode, B, S, max_seq):
    lay = synth.make_layer(R1, "fake")
    with mode:
        aw = {k: (tuple(mode.from_tensor(t).to("cuda") for t in v) if isinstance(v, tuple)
                  else mode.from_tensor(v).to("cuda")) for k, v in lay.attn_weights.items()}
        h = torch.empty(B, S, R1.hidden_size, dtype=torch.bfloat16, device="cuda")
        ckv = torch.empty(B, max_seq, 512, dtype=torch.bfloat16, device="cuda")
        kpe = torch.empty(B, max_seq, 64, dtype=torch.bfloat16, device="cuda")
        tab = torch.empty(max_seq, 32, dtype=torch.complex64, device="cuda")
    return aw, h, ckv, kpe, tab


def test_mla_attention_traces_under_fake_tensors():
    mode = FakeTensorMode()
    for S, op in ((1, "mla_decode"), (5, "mla_prefill")):
        aw, h, ckv, kpe, tab = _fake_inputs(mode, 2, S, 64)
        with mode:
            out = ops.mla_attention(h, aw, (ckv, kpe), 7, tab, R1)
        assert out.shape == (2, S, R1.hidden_size) and out.dtype == torch.bfloat16

        def f(h, ckv, kpe, tab):
            return ops.mla_attention(h, aw, (ckv, kpe), 7, tab, R1)

        gm = make_fx(f, tracing_mode="fake")(h, ckv, kpe, tab)
        targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
        assert f"amla.{op}.default" in targets, targets


def test_functionalized_trace_keeps_the_cache_write():
    """Under functionalization (what torch.compile and torch.export run) the in-place cache
    store (inference/ops.py:140-141) becomes an explicit functional op over both caches."""
    mode = FakeTensorMode()
    aw, h, ckv, kpe, tab = _fake_inputs(mode, 1, 1, 16)

    def f(h, ckv, kpe, tab):
        return ops.mla_attention(h, aw, (ckv, kpe), 3, tab, R1)

    gm = make_fx(dispatch_functionalize(f), tracing_mode="fake")(h, ckv, kpe, tab)
    code = gm.code
    assert "auto_functionalized" in code and "amla.mla_decode" in code, code
    # both caches are tracked as mutated bases of the functional op
    assert "_ckv_cache_base_index = 0" in code and "_kpe_cache_base_index = 1" in code, code


def test_linear_norm_rope_fake_shapes():
    mode = FakeTensorMode()
    with mode:
        x = torch.empty(3, 1, 7168, dtype=torch.bfloat16, device="cuda")
        w = torch.empty(1536, 7168, dtype=torch.float8_e4m3fn, device="cuda")
        s = torch.empty(12, 56, dtype=torch.float32, device="cuda")
        y = ops.fp8_linear(x, w, s)
        y32 = ops.fp8_linear(x, w, s, out_dtype=torch.float32)
        y16 = ops.fp8_linear(x, w, s, out_dtype=torch.float16)
        gu = torch.empty(256, 7168, dtype=torch.float8_e4m3fn, device="cuda")
        gs = torch.empty(2, 56, dtype=torch.float32, device="cuda")
        dw = torch.empty(7168, 256, dtype=torch.float8_e4m3fn, device="cuda")
        ds = torch.empty(56, 2, dtype=torch.float32, device="cuda")
        sw = ops.swiglu(x, gu, gs, gu, gs, dw, ds)
        g = torch.empty(7168, dtype=torch.bfloat16, device="cuda")
        n = ops.rms_norm(x, g)
        q = torch.empty(2, 128, 4, 64, dtype=torch.bfloat16, device="cuda")
        f = torch.empty(4, 32, dtype=torch.complex64, device="cuda")
        r = ops.apply_rope(q, f)
    assert y.shape == (3, 1, 1536) and n.shape == x.shape and r.shape == q.shape
    assert y32.dtype == torch.float32 and y16.dtype == torch.float16 and y32.shape == y.shape
    assert sw.shape == x.shape and sw.dtype == torch.bfloat16


def test_shims_read_no_data_pointer_of_fake_tensors():
    """Alignment is checked inside the operators, on real tensors: tracing the linear and the
    SwiGLU shims under FakeTensorMode warns about no data-pointer access."""
    import warnings
    mode = FakeTensorMode()
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        with mode:
            x = torch.empty(2, 7168, dtype=torch.bfloat16, device="cuda")[:, :7168]
            w = torch.empty(1536, 7168, dtype=torch.float8_e4m3fn, device="cuda")
            s = torch.empty(12, 56, dtype=torch.float32, device="cuda")
            ops.fp8_linear(x, w, s)
            gu = torch.empty(256, 7168, dtype=torch.float8_e4m3fn, device="cuda")
            gs = torch.empty(2, 56, dtype=torch.float32, device="cuda")
            ops.swiglu(x, gu, gs, gu, gs, torch.empty(7168, 256, dtype=torch.float8_e4m3fn, device="cuda"),
                       torch.empty(56, 2, dtype=torch.float32, device="cuda"))
