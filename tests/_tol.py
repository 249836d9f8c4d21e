"""Parity bars shared by the GPU tests.

bf16 outputs against the oracle (oracle/ref_ops.py, the reference's rounding
points):
* elementwise |gpu - oracle| <= ATOL + RTOL * |oracle|, ATOL = RTOL = 2e-2
  (the bar the path is specified with);
* normwise max|delta| / max|oracle| <= 2e-2;
* RMS: rms(gpu - oracle) / rms(oracle) <= RMS_MAX = 1e-2.  The elementwise bar
  alone is loose for attention outputs (std 0.03-0.09), the RMS bar is not.

Per-head attention outputs (before o_proj, (.., heads * v_dim)): the same bars
per head, so that a fault confined to one of 128 heads cannot hide behind
o_proj's mixing.

Against float64 truth (oracle/truth.py): the GPU's RMS error is at most
TRUTH_FACTOR = 2 times the oracle's own RMS error.  The oracle rounds scores
and probabilities to bf16 where the kernels keep fp32, so a correct kernel is
usually closer to the truth than the oracle; a dropped term, a wrong sign or a
misplaced row is not.
"""
import torch

ATOL = 2e-2
RTOL = 2e-2
NORMWISE_MAX = 2e-2
RMS_MAX = 1e-2
TRUTH_FACTOR = 2.0


def _rms(t: torch.Tensor) -> float:
    return t.double().pow(2).mean().sqrt().item() if t.numel() else 0.0


def report(got: torch.Tensor, ref: torch.Tensor) -> dict:
    g, r = got.detach().float().cpu(), ref.detach().float().cpu()
    d = (g - r).abs()
    return {
        "max_abs": d.max().item(),
        "normwise": (d.max() / r.abs().max().clamp_min(1e-30)).item(),
        "rms_ratio": _rms(d) / max(_rms(r), 1e-30),
        "bit_identical": (g == r).float().mean().item(),
        "worst_excess": (d - (ATOL + RTOL * r.abs())).max().item(),
    }


def assert_parity(got: torch.Tensor, ref: torch.Tensor, what: str = "", atol=ATOL, rtol=RTOL, rms_max=RMS_MAX):
    g, r = got.detach().float().cpu(), ref.detach().float().cpu()
    assert g.shape == r.shape, (what, g.shape, r.shape)
    assert torch.isfinite(g).all(), f"{what}: non-finite output"
    rep = report(g, r)
    ok = ((g - r).abs() <= atol + rtol * r.abs()).all().item()
    assert ok and rep["normwise"] <= NORMWISE_MAX and rep["rms_ratio"] <= rms_max, f"{what}: {rep}"
    print(f"[parity] {what}: {rep}", flush=True)
    return rep


def assert_heads_parity(got: torch.Tensor, ref: torch.Tensor, heads: int, what: str = "", rms_max=RMS_MAX):
    """Per-head bars on (..., heads * v) attention outputs: every head's RMS ratio,
    normwise ratio and elementwise bound, plus the whole tensor."""
    g = got.detach().float().cpu().reshape(-1, heads, got.shape[-1] // heads)
    r = ref.detach().float().cpu().reshape(-1, heads, ref.shape[-1] // heads)
    assert g.shape == r.shape and torch.isfinite(g).all(), what
    d = g - r
    rms_h = d.double().pow(2).mean((0, 2)).sqrt() / r.double().pow(2).mean((0, 2)).sqrt().clamp_min(1e-30)
    norm_h = d.abs().amax((0, 2)) / r.abs().amax((0, 2)).clamp_min(1e-30)
    elem_ok = (d.abs() <= ATOL + RTOL * r.abs()).all().item()
    worst = int(rms_h.argmax())
    msg = (f"{what}: worst head {worst} rms {rms_h[worst].item():.3e}, max normwise {norm_h.max().item():.3e}, "
           f"elementwise ok {elem_ok}")
    assert elem_ok and rms_h.max().item() <= rms_max and norm_h.max().item() <= NORMWISE_MAX, msg
    print(f"[heads] {msg}", flush=True)
    return rms_h


def assert_closer_than(got: torch.Tensor, oracle: torch.Tensor, truth: torch.Tensor, what: str = "",
                       factor: float = TRUTH_FACTOR):
    """rms(got - truth) <= factor * rms(oracle - truth) (+ a floor of 1e-6 rms(truth))."""
    g, o, t = got.detach().double().cpu(), oracle.detach().double().cpu(), truth.detach().double().cpu()
    eg, eo = _rms(g - t), _rms(o - t)
    floor = 1e-6 * _rms(t)
    assert eg <= factor * eo + floor, f"{what}: gpu rms error {eg:.3e} > {factor} x oracle's {eo:.3e}"
    print(f"[truth] {what}: gpu rms err {eg:.3e}, oracle rms err {eo:.3e} (ratio {eg / max(eo, 1e-300):.3f})",
          flush=True)
    return eg, eo


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
