"""Parity bar shared by the GPU tests.

bf16 outputs: |gpu - oracle| <= ATOL + RTOL * |oracle| elementwise, with
ATOL = RTOL = 2e-2, and the normwise max|delta| / max|oracle| <= 2e-2.
The oracle (oracle/ref_ops.py) keeps the reference's bf16 rounding points
(including bf16 attention scores), so an fp32-score kernel differs from it by
the oracle's own rounding; the relative term covers large linear outputs where
one bf16 ulp already exceeds 2e-2.
"""
import torch

ATOL = 2e-2
RTOL = 2e-2


def report(got: torch.Tensor, ref: torch.Tensor) -> dict:
    g, r = got.detach().float().cpu(), ref.detach().float().cpu()
    d = (g - r).abs()
    return {
        "max_abs": d.max().item(),
        "normwise": (d.max() / r.abs().max().clamp_min(1e-30)).item(),
        "rms_ratio": (d.pow(2).mean().sqrt() / r.pow(2).mean().sqrt().clamp_min(1e-30)).item(),
        "bit_identical": (g == r).float().mean().item(),
        "worst_excess": (d - (ATOL + RTOL * r.abs())).max().item(),
    }


def assert_parity(got: torch.Tensor, ref: torch.Tensor, what: str = "", atol=ATOL, rtol=RTOL):
    rep = report(got, ref)
    g, r = got.detach().float().cpu(), ref.detach().float().cpu()
    assert g.shape == r.shape, (what, g.shape, r.shape)
    assert torch.isfinite(g).all(), f"{what}: non-finite output"
    ok = ((g - r).abs() <= atol + rtol * r.abs()).all().item()
    assert ok and rep["normwise"] <= 2e-2, f"{what}: {rep}"
    print(f"[parity] {what}: {rep}", flush=True)
    return rep


def assert_bf16_ulps(got: torch.Tensor, ref: torch.Tensor, ulps: int, what: str = "", abs_floor: float = 1e-3):
    """|got - ref| <= ulps * 2^-7 * |ref| + abs_floor elementwise: within `ulps`
    bf16 units in the last place of the reference, except for values so close
    to zero (fp32 sums that cancel) that an absolute floor is the only
    meaningful scale."""
    g = got.detach().float().cpu()
    r = ref.detach().float().cpu()
    d = (g - r).abs()
    bound = ulps * 2.0 ** -7 * r.abs() + abs_floor
    worst = (d / bound).max().item() if d.numel() else 0.0
    assert worst <= 1.0, f"{what}: {worst:.2f} x the {ulps}-ulp bound (max |d| {d.max().item():.3e})"
    return worst
