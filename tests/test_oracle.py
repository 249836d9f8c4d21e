"""Pins the CPU oracle (oracle/) against golden vectors, closed forms and invariants.

No GPU.  Golden vectors were written by tests/golden/make_golden.py from the
reference's own inference/ops.py.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from oracle import ref_ops as R
from oracle import truth as T
from amla import synth
from amla.config import DeepSeekConfig

SMALL = dict(hidden_size=320, num_attention_heads=4, q_lora_rank=192, kv_lora_rank=160,
             qk_nope_head_dim=48, qk_rope_head_dim=16, v_head_dim=40, qk_head_dim=64)


def _bf16(bits):
    return bits.view(torch.bfloat16)


# ---------------------------------------------------------------- fp8 decode / dequant

def _ocp_e4m3(code: int) -> float:
    """Textbook OCP e4m3fn value, computed independently of oracle/fp8_ref.c."""
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 7
    if e == 15 and m == 7:
        return float("nan")
    if e == 0:
        return s * m * 2.0 ** -9
    return s * (1 + m / 8) * 2.0 ** (e - 7)


def test_e4m3_table_all_codes():
    table = oracle.c_e4m3_table()
    torch_dec = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    for c in range(256):
        want = _ocp_e4m3(c)
        if math.isnan(want):
            assert np.isnan(table[c]) and np.isnan(torch_dec[c])
        else:
            assert table[c] == np.float32(want), c
            assert table[c].view(np.uint32) == torch_dec[c].view(np.uint32), c  # signed zero too
    assert table[0x7E] == 448.0 and table[0x01] == 2.0 ** -9 and table[0x38] == 1.0
    assert table[0x80].view(np.uint32) == 0x80000000  # -0.0 kept


@pytest.mark.parametrize("N,K", [(300, 200), (576, 256), (128, 128), (1, 7)])
def test_block_dequant_matches_c_restatement(N, K):
    g = torch.Generator().manual_seed(N * 1000 + K)
    codes = torch.randint(0, 256, (N, K), generator=g, dtype=torch.uint8)
    codes[codes == 0x7F] = 0x7E
    codes[codes == 0xFF] = 0xFE
    w = codes.view(torch.float8_e4m3fn)
    sc = torch.exp(torch.randn(math.ceil(N / 128), math.ceil(K / 128), generator=g) * 4).float()
    got = R.fp8_block_dequant(w, sc).numpy()
    want = oracle.c_fp8_block_dequant(codes.numpy(), sc.numpy())
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_block_dequant_partial_row_block():
    # wkv_a: 576 rows -> scale rows 0..4, row block 4 covers rows 512..575 only
    codes = torch.full((576, 256), 0x38, dtype=torch.uint8)  # all 1.0
    sc = torch.arange(10, dtype=torch.float32).view(5, 2) + 1
    got = R.fp8_block_dequant(codes.view(torch.float8_e4m3fn), sc)
    assert torch.all(got[512:, :128] == 9.0) and torch.all(got[512:, 128:] == 10.0)
    assert torch.all(got[:128, :128] == 1.0)


def test_quantizer_roundtrip_and_clamp():
    w = synth.randn((256, 384), 7, 0.02)
    w[3, 5] = 1.0                                  # dominates its block
    q, s = synth.quantize_fp8_blocks(w)
    assert s.shape == (2, 3) and q.dtype == torch.float8_e4m3fn
    deq = R.fp8_block_dequant(q, s)
    assert not torch.isnan(deq).any()
    assert deq[3, 5] == pytest.approx(1.0, rel=1e-6)   # amax maps to exactly 448 * scale
    blockwise = (w - deq).abs().view(2, 128, 3, 128).amax((1, 3))
    assert torch.all(blockwise <= s * 16 + 1e-12)       # half-ulp of e4m3 at 448 is 16


# ---------------------------------------------------------------- fp8_linear

def test_fp8_linear_vs_fp64_bruteforce():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(5, 300, generator=g).to(torch.bfloat16)
    w, s = synth.quantize_fp8_blocks(synth.randn((200, 300), 11, 0.02))
    y = R.fp8_linear(x, w, s)
    ref = x.double() @ R.fp8_block_dequant(w, s).double().T
    assert y.dtype == torch.bfloat16
    assert torch.allclose(y.double(), ref, rtol=2 ** -8, atol=1e-6)


def test_fp8_linear_identity_is_exact():
    x = torch.randn(3, 128).to(torch.bfloat16)
    w = torch.eye(128).to(torch.float8_e4m3fn)
    y = R.fp8_linear(x, w, torch.ones(1, 1))
    assert torch.equal(y, x)
    # one-hot rows with a power-of-two scale select and scale exactly
    idx = torch.randperm(128)
    w1 = torch.zeros(128, 128)
    w1[torch.arange(128), idx] = 1.0
    y = R.fp8_linear(x, w1.to(torch.float8_e4m3fn), torch.full((1, 1), 0.25))
    assert torch.equal(y, (x[:, idx].float() * 0.25).to(torch.bfloat16))


# ---------------------------------------------------------------- rms_norm

def test_rms_norm_closed_forms():
    x = torch.full((2, 64), 3.0).to(torch.bfloat16)
    y = R.rms_norm(x, torch.ones(64, dtype=torch.bfloat16))
    assert torch.allclose(y.float(), torch.ones(2, 64), atol=2 ** -8)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(4, 512, generator=g).to(torch.bfloat16)
    gam = (1 + 0.1 * torch.randn(512, generator=g)).to(torch.bfloat16)
    r = 1.0 / np.sqrt((x.double() ** 2).mean(-1, keepdim=True).numpy() + 1e-6)
    want = (torch.from_numpy(x.double().numpy() * r).to(torch.bfloat16) * gam)
    got = R.rms_norm(x, gam, 1e-6)
    assert got.dtype == torch.bfloat16
    d = (got.float() - want.float()).abs() / want.float().abs().clamp_min(1e-3)
    assert d.max() <= 2 ** -7   # at most one bf16 ulp apart (fp32 vs fp64 rsqrt)


# ---------------------------------------------------------------- YaRN scalars and table

def test_yarn_scalars():
    cfg = DeepSeekConfig()
    ms = R.yarn_get_mscale(cfg.rope_scaling_factor, cfg.rope_scaling_mscale_all_dim)
    assert ms == pytest.approx(0.1 * math.log(40) + 1, abs=0) and ms == pytest.approx(1.3688879454113936, abs=1e-15)
    assert R.yarn_get_mscale(1.0, 1.0) == 1.0 and R.yarn_get_mscale(0.5, 3.0) == 1.0
    assert ms / math.sqrt(192) == pytest.approx(0.09879097797171274, abs=1e-15)
    assert R.yarn_ramp_bounds(cfg) == (10, 23)


def test_rope_table_matches_reference(golden):
    tens, man = golden
    cfg = DeepSeekConfig()
    tab = R.precompute_rope_freqs(cfg, man["rope"]["seq_len"])
    rows = tens["rope.rows"].tolist()
    got = torch.view_as_real(tab[rows])
    assert torch.equal(got.view(torch.int32), tens["rope.table_rows"].view(torch.int32))
    assert torch.equal(torch.view_as_real(tab[:64]), tens["rope.table_0_64"])


def test_rope_table_closed_forms():
    cfg = DeepSeekConfig()
    tab = R.precompute_rope_freqs(cfg, 4096)
    assert torch.allclose(tab.abs(), torch.ones(()), atol=1e-6)
    f = R.yarn_inv_freq(cfg).double()
    textbook = 1.0 / (10000.0 ** (torch.arange(0, 64, 2, dtype=torch.float64) / 64))
    assert torch.allclose(f[:10], textbook[:10], rtol=1e-6)            # below low: unscaled
    assert torch.allclose(f[24:], textbook[24:] / 40, rtol=1e-6)       # above high: /factor
    cfg1 = DeepSeekConfig(rope_scaling_factor=1.0)
    assert torch.allclose(R.yarn_inv_freq(cfg1).double(), textbook, rtol=1e-6)
    t = 1000
    assert torch.allclose(torch.angle(tab[t]).double(), torch.remainder(t * f + math.pi, 2 * math.pi) - math.pi,
                          atol=2e-3)


def test_apply_rope_matches_reference(golden):
    tens, man = golden
    cfg = DeepSeekConfig()
    tab = R.precompute_rope_freqs(cfg, 32768)
    x = _bf16(tens["apply_rope.x"])
    for name in ("p0", "p300", "p32760"):
        s = man[f"apply_rope.{name}"]["start"]
        y = R.apply_rope(x, tab[s:s + 5])
        assert torch.equal(y.view(torch.int16), tens[f"apply_rope.{name}.y"]), name
    # position 0 rotates by angle 0: identity
    y0 = R.apply_rope(x[:, :, :1], tab[:1])
    assert torch.equal(y0, x[:, :, :1])


# ---------------------------------------------------------------- mla_attention

def _rebuild(man_entry):
    cfg = DeepSeekConfig(**man_entry["cfg"])
    tag = man_entry["tag"]
    lay = synth.make_layer(cfg, tag)
    hidden = synth.make_hidden(cfg, man_entry["B"], man_entry["S"], tag)
    ckv, kpe = synth.make_kv_cache(cfg, man_entry["B"], man_entry["max_seq"], man_entry["filled"], tag)
    return cfg, lay, hidden, ckv, kpe


@pytest.mark.parametrize("key", ["small_decode", "small_prefill", "small_chunk", "r1_decode_t257", "r1_prefill_s8"])
def test_mla_attention_matches_reference(golden, key):
    tens, man = golden
    e = man[key]
    cfg, lay, hidden, ckv, kpe = _rebuild(e)
    assert synth.sha256_of(hidden) == e["sha256"]["hidden"]
    assert synth.sha256_of(lay.attn_weights["o_proj"][0]) == e["sha256"]["o_proj"]
    tab = R.precompute_rope_freqs(cfg, e["max_seq"])
    y = R.mla_attention(hidden, lay.attn_weights, (ckv, kpe), e["position"], tab, cfg)
    p, S = e["position"], e["S"]
    assert torch.equal(ckv[:, p:p + S].view(torch.int16), tens[f"{key}.ckv_new"])
    assert torch.equal(kpe[:, p:p + S].view(torch.int16), tens[f"{key}.kpe_new"])
    want = _bf16(tens[f"{key}.out"])
    assert torch.equal(y.view(torch.int16), want.view(torch.int16)), (y - want).abs().max()


def test_naive_equals_absorbed_fp64():
    cfg = DeepSeekConfig(**SMALL)
    lay = synth.make_layer(cfg, "absorb")
    B, max_seq = 3, 24
    positions = [5, 17, 0]
    ckv, kpe = synth.make_kv_cache(cfg, B, max_seq, [p + 1 for p in positions], "absorb")
    hidden = synth.make_hidden(cfg, B, 1, "absorb")
    tab = R.precompute_rope_freqs(cfg, max_seq)
    ab = T.mla_decode_absorbed_f64(hidden, lay.attn_weights, ckv, kpe, positions, tab, cfg)
    for b, p in enumerate(positions):
        nv = T.mla_naive_f64(hidden[b:b + 1], lay.attn_weights, ckv[b:b + 1], kpe[b:b + 1], p, tab, cfg)
        assert torch.allclose(ab[b], nv[0], rtol=1e-10, atol=1e-12)


def test_single_position_ignores_query():
    # T = 1: softmax is 1, so the output does not depend on the query weights
    cfg = DeepSeekConfig(**SMALL)
    lay = synth.make_layer(cfg, "t1")
    ckv, kpe = synth.make_kv_cache(cfg, 1, 4, 1, "t1")
    hidden = synth.make_hidden(cfg, 1, 1, "t1")
    tab = R.precompute_rope_freqs(cfg, 4)
    a = T.mla_naive_f64(hidden, lay.attn_weights, ckv, kpe, 0, tab, cfg)
    aw2 = dict(lay.attn_weights)
    w, s = aw2["q_b_proj"]
    aw2["q_b_proj"] = (w, s * 3.0)
    b = T.mla_naive_f64(hidden, aw2, ckv, kpe, 0, tab, cfg)
    assert torch.allclose(a, b, rtol=1e-12)


def test_uniform_rows_give_uniform_attention():
    cfg = DeepSeekConfig(**SMALL)
    lay = synth.make_layer(cfg, "uni")
    ckv, kpe = synth.make_kv_cache(cfg, 1, 8, 1, "uni")
    ckv[0, 1:6] = ckv[0, 0]
    kpe[0, :6] = 0
    hidden = synth.make_hidden(cfg, 1, 1, "uni")
    tab = R.precompute_rope_freqs(cfg, 8)
    a = T.mla_naive_f64(hidden, lay.attn_weights, ckv, kpe, 5, tab, cfg)
    ckv1, kpe1 = ckv.clone(), kpe.clone()
    b = T.mla_naive_f64(hidden, lay.attn_weights, ckv1[:, :1], kpe1[:, :1], 0, tab, cfg)
    assert torch.allclose(a, b, rtol=1e-10)


def test_oracle_within_tolerance_of_truth():
    cfg = DeepSeekConfig(**SMALL)
    lay = synth.make_layer(cfg, "budget")
    ckv, kpe = synth.make_kv_cache(cfg, 2, 40, 33, "budget")
    hidden = synth.make_hidden(cfg, 2, 1, "budget")
    tab = R.precompute_rope_freqs(cfg, 40)
    y = R.mla_attention(hidden, lay.attn_weights, (ckv.clone(), kpe.clone()), 33, tab, cfg)
    ckv[:, 33:34] = R.fp8_linear(hidden, *lay.attn_weights["kv_a_proj_with_mqa"])[..., :160]
    kpe[:, 33:34] = R.fp8_linear(hidden, *lay.attn_weights["kv_a_proj_with_mqa"])[..., 160:]
    t = T.mla_naive_f64(hidden, lay.attn_weights, ckv, kpe, 33, tab, cfg)
    err = (y.double() - t).abs()
    assert torch.all(err <= 2e-2 + 2e-2 * t.abs())


def test_absorbed_heads_equal_naive_heads_fp64():
    """The per-head outputs (before o_proj) of the absorbed and naive fp64 forms agree."""
    cfg = DeepSeekConfig(**SMALL)
    lay = synth.make_layer(cfg, "absorb-heads")
    positions = [9, 2]
    ckv, kpe = synth.make_kv_cache(cfg, 2, 16, [p + 1 for p in positions], "absorb-heads")
    hidden = synth.make_hidden(cfg, 2, 1, "absorb-heads")
    tab = R.precompute_rope_freqs(cfg, 16)
    heads, out = T.mla_decode_absorbed_parts_f64(hidden, lay.attn_weights, ckv, kpe, positions, tab, cfg)
    for b, p in enumerate(positions):
        nh, no = T.mla_naive_parts_f64(hidden[b:b + 1], lay.attn_weights, ckv[b:b + 1], kpe[b:b + 1], p, tab, cfg)
        assert torch.allclose(heads[b], nh[0], rtol=1e-10, atol=1e-12)
        assert torch.allclose(out[b], no[0], rtol=1e-10, atol=1e-12)
    # o_proj of the heads is the output (the split of the two parts is where ops.py:182-183 puts it)
    assert torch.allclose(heads @ T._w64(lay.attn_weights["o_proj"]).T, out, rtol=1e-12)


def test_prefill_rows_f64_equal_naive_prefill():
    """mla_prefill_rows_f64 (absorbed, per query row) equals rows of the naive fp64 causal prefill,
    including a first position > 0 (a chunk after cached rows)."""
    cfg = DeepSeekConfig(**SMALL)
    lay = synth.make_layer(cfg, "rows")
    S, p = 7, 4
    ckv, kpe = synth.make_kv_cache(cfg, 1, 16, p + S, "rows")
    hidden = synth.make_hidden(cfg, 1, S, "rows")
    tab = R.precompute_rope_freqs(cfg, 16)
    nh, no = T.mla_naive_parts_f64(hidden, lay.attn_weights, ckv, kpe, p, tab, cfg)
    rows = [0, 3, 6]
    h, o = T.mla_prefill_rows_f64(hidden, lay.attn_weights, ckv, kpe, p, rows, tab, cfg)
    assert torch.allclose(h, nh[0, rows], rtol=1e-10, atol=1e-12)
    assert torch.allclose(o, no[0, rows], rtol=1e-10, atol=1e-12)


def test_parts_final_is_o_proj_of_heads(golden):
    """mla_attention_parts: the final output is fp8_linear(heads, o_proj), equal to the
    reference's own output bit for bit (golden vector), so the heads tensor is the
    reference's pre-o_proj activation."""
    tens, man = golden
    e = man["r1_decode_t257"]
    cfg, lay, hidden, ckv, kpe = _rebuild(e)
    tab = R.precompute_rope_freqs(cfg, e["max_seq"])
    heads, out = R.mla_attention_parts(hidden, lay.attn_weights, (ckv, kpe), e["position"], tab, cfg)
    assert heads.shape == (1, 1, cfg.num_attention_heads * cfg.v_head_dim)
    assert torch.equal(R.fp8_linear(heads, *lay.attn_weights["o_proj"]).view(torch.int16), out.view(torch.int16))
    assert torch.equal(out.view(torch.int16), tens["r1_decode_t257.out"])
