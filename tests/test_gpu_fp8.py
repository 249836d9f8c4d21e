"""GPU parity of the block-FP8 kernels and the small ops against the oracle."""
import math

import numpy as np
import pytest
import torch

import oracle
from oracle import ref_ops as R
from amla import ops, synth
from amla.config import DeepSeekConfig
from _tol import assert_parity, assert_bf16_ulps

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
R1 = DeepSeekConfig()
SHAPES = synth.projection_shapes(R1)


def _w(name, seed_tag="fp8"):
    n, k = SHAPES[name]
    return synth.quantize_fp8_blocks(synth.randn((n, k), synth.seed_of(seed_tag, name), 0.02))


def test_dequant_all_codes_bit_exact():
    codes = torch.arange(256, dtype=torch.uint8).repeat(300, 2)[:, :384].contiguous()   # (300, 384)
    g = torch.Generator().manual_seed(1)
    sc = torch.exp(torch.randn(3, 3, generator=g) * 6).float()
    sc[0, 0] = 1.0
    got = ops.fp8_block_dequant(codes.view(torch.float8_e4m3fn).to(DEV), sc.to(DEV)).cpu().numpy()
    want = oracle.c_fp8_block_dequant(codes.numpy(), sc.numpy())
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got.view(np.uint32)[~nan], want.view(np.uint32)[~nan])


@pytest.mark.parametrize("name", list(SHAPES))
def test_dequant_r1_weights_bit_exact(name):
    w, s = _w(name)
    got = ops.fp8_block_dequant(w.to(DEV), s.to(DEV)).cpu()
    want = R.fp8_block_dequant(w, s)
    assert torch.equal(got.view(torch.int32), want.view(torch.int32)), name


@pytest.mark.parametrize("name", list(SHAPES))
@pytest.mark.parametrize("M", [1, 2, 5, 8, 17, 32, 64])
def test_fp8_linear_r1_shapes(name, M):
    """M = 1 takes the streaming GEMVs, 2-8 the GEMV with x in LDS at these shapes (masked
    columns past M), 9-64 the skinny GEMM (one, two or four 16-row x tiles in registers)."""
    print(f"[case] fp8_linear {name} M={M}", flush=True)
    w, s = _w(name)
    x = synth.randn((M, SHAPES[name][1]), synth.seed_of("fp8x", name, M)).to(torch.bfloat16)
    got = ops.fp8_linear(x.to(DEV), w.to(DEV), s.to(DEV))
    torch.cuda.synchronize()
    want = R.fp8_linear(x, w, s)
    assert_parity(got, want, f"fp8_linear {name} M={M}")
    assert_bf16_ulps(got, want, 2, f"fp8_linear {name} M={M}")


@pytest.mark.parametrize("M,name", [(4096, "q_a_proj"), (300, "o_proj"), (65, "kv_b_proj"), (200, "kv_a_proj_with_mqa")])
def test_fp8_linear_large_m(M, name):
    print(f"[case] fp8_linear large {name} M={M}", flush=True)
    w, s = _w(name)   # kv_a: 576 rows, the last 128-row scale block is partial
    x = synth.randn((M, SHAPES[name][1]), synth.seed_of("fp8xl", name, M)).to(torch.bfloat16)
    got = ops.fp8_linear(x.to(DEV), w.to(DEV), s.to(DEV))
    want = R.fp8_linear(x, w, s)
    assert_parity(got, want, f"fp8_linear {name} M={M}")
    assert_bf16_ulps(got, want, 2, f"fp8_linear {name} M={M}")


@pytest.mark.parametrize("name,M", [("q_b_proj", 1), ("o_proj", 8), ("kv_b_proj", 64), ("q_a_proj", 100),
                                    ("kv_a_proj_with_mqa", 300)])
def test_fp8_linear_out_dtype(name, M):
    """out_dtype (inference/ops.py:19, :44): fp32 is the unrounded fp32 result, within fp32
    summation-order error of the oracle's (a dropped 128-wide block or a wrong scale would miss by
    about 1/128 of the magnitude sum); float16 is that result cast, as the reference casts it."""
    print(f"[case] fp8_linear out_dtype {name} M={M}", flush=True)
    w, s = _w(name)
    x = synth.randn((M, SHAPES[name][1]), synth.seed_of("fp8x32", name, M)).to(torch.bfloat16)
    got = ops.fp8_linear(x.to(DEV), w.to(DEV), s.to(DEV), out_dtype=torch.float32)
    got16 = ops.fp8_linear(x.to(DEV), w.to(DEV), s.to(DEV), out_dtype=torch.float16)
    torch.cuda.synchronize()
    assert got.dtype == torch.float32 and got.shape == (M, SHAPES[name][0])
    want = R.fp8_linear(x, w, s, out_dtype=torch.float32)
    mag = x.float().abs() @ R.fp8_block_dequant(w, s).abs().T
    err = (got.cpu() - want).abs()
    assert (err <= 2.0 ** -16 * mag).all(), f"max err {err.max().item():.3e}"
    assert got16.dtype == torch.float16
    assert torch.equal(got16.cpu(), got.cpu().to(torch.float16))


@pytest.mark.parametrize("N,K", [(160, 1536), (208, 1536), (32, 4096), (1040, 7168), (4112, 16384)])
def test_fp8_linear_streaming_ragged_rows(N, K):
    """One row of x takes the streaming GEMVs (K = 1536, and 4096 <= K <= 16384): row counts
    that leave the last workgroup's run of rows partial, and partial 128-row scale blocks."""
    print(f"[case] fp8_linear streaming N={N} K={K}", flush=True)
    w, s = synth.quantize_fp8_blocks(synth.randn((N, K), synth.seed_of("fp8vs", N, K), 0.02))
    x = synth.randn((1, K), synth.seed_of("fp8vsx", N, K)).to(torch.bfloat16)
    got = ops.fp8_linear(x.to(DEV), w.to(DEV), s.to(DEV))
    torch.cuda.synchronize()
    want = R.fp8_linear(x, w, s)
    assert_parity(got, want, f"fp8_linear streaming N={N} K={K}")
    assert_bf16_ulps(got, want, 2, f"fp8_linear streaming N={N} K={K}")


def test_fp8_linear_repeat_is_deterministic():
    w, s = _w("o_proj")
    x = synth.randn((8, SHAPES["o_proj"][1]), 5).to(torch.bfloat16).to(DEV)
    a = ops.fp8_linear(x, w.to(DEV), s.to(DEV))
    b = ops.fp8_linear(x, w.to(DEV), s.to(DEV))
    assert torch.equal(a, b)


@pytest.mark.parametrize("rows,dim", [(1, 1536), (8, 7168), (4096, 512), (3, 200)])
def test_rms_norm(rows, dim):
    x = synth.randn((rows, dim), synth.seed_of("rms", rows, dim)).to(torch.bfloat16)
    gam = synth.gamma(dim, synth.seed_of("rmsg", dim))
    got = ops.rms_norm(x.to(DEV), gam.to(DEV), 1e-6).cpu()
    want = R.rms_norm(x, gam, 1e-6)
    assert_bf16_ulps(got, want, 1, f"rms_norm {rows}x{dim}")


def test_apply_rope_matches_oracle():
    tab = R.precompute_rope_freqs(R1, 4096)
    x = synth.randn((2, 128, 7, 64), 9).to(torch.bfloat16)
    for start in (0, 255, 4089):
        f = tab[start:start + 7]
        got = ops.apply_rope(x.to(DEV), f.to(DEV)).cpu()
        want = R.apply_rope(x, f)
        assert_bf16_ulps(got, want, 1, f"apply_rope start={start}")


def test_rope_table_matches_oracle():
    got = ops.precompute_rope_freqs(R1, 4096, DEV).cpu()
    want = R.precompute_rope_freqs(R1, 4096)
    assert torch.equal(torch.view_as_real(got), torch.view_as_real(want))
