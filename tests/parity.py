"""Comparison helpers shared by the parity tests."""

from __future__ import annotations

import torch

# The build's numerical contract: fp32 states and bf16 outputs within rtol = atol = 2e-3 of
# the oracle (after 64 recurrent steps where the workload says so).
RTOL = 2e-3
ATOL = 2e-3
# The reference's own output tolerance (tests/test_gdn.py:73), which must hold everywhere.
REF_OUT_ATOL = 0.008
REF_OUT_RTOL = 0.02
# A bf16 rounding of an fp32 value within this fraction of a bf16 ulp of the midpoint
# between two bf16 neighbours can legitimately go either way under a different (but
# equally valid) fp32 summation order.
MIDPOINT_WINDOW = 0.05
# Such rounding-sensitive elements may differ by at most this many bf16 ulps ...
MAX_FLIP_ULPS = 2
# ... and may make up at most this fraction of the compared elements.
MAX_FLIP_FRACTION = 2e-3


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bfloat16 numbers at |x| (fp32 tensor)."""
    mag = x.float().abs().clamp_min(2.0**-126)
    exponent = torch.floor(torch.log2(mag))
    return torch.pow(2.0, exponent - 7)


def near_bf16_midpoint(x: torch.Tensor, window: float = MIDPOINT_WINDOW) -> torch.Tensor:
    """True where fp32 `x` lies within `window` bf16 ulps of a bf16 rounding midpoint."""
    low16 = (x.float().contiguous().view(torch.int32) & 0xFFFF).float() / 65536.0
    return (low16 - 0.5).abs() < window


def rstd_shift_ulps(raw_pre: torch.Tensor, y_pre: torch.Tensor,
                    window: float = MIDPOINT_WINDOW) -> torch.Tensor:
    """How far (in bf16 ulps of y) each y = bf16(raw) * rsqrt(mean(bf16(raw)^2) + eps) * ...
    can move when the rounding-sensitive raw elements of its row (last dimension) round the
    other way: such a flip changes the row's mean square, hence every y of the row.  The
    bound leaves eps out of the mean square, which only enlarges it."""
    raw = raw_pre.float()
    low = raw.bfloat16().float()
    ulp = bf16_ulp(raw)
    other = torch.where(raw >= low, low + ulp, low - ulp)  # the neighbour across the midpoint
    sensitive = near_bf16_midpoint(raw, window)
    delta = torch.where(sensitive, (other.square() - low.square()).abs(), torch.zeros_like(raw))
    ms = low.square().sum(-1, keepdim=True)
    rel = 0.5 * delta.sum(-1, keepdim=True) / ms.clamp_min(torch.finfo(torch.float32).tiny)
    y = y_pre.float()
    return rel * y.abs() / bf16_ulp(y)


def assert_bf16_outputs(actual: torch.Tensor, expected: torch.Tensor, pre=None, *,
                        rtol: float = RTOL, atol: float = ATOL, label: str = "out") -> dict:
    """bf16 outputs within rtol/atol of the oracle, except elements whose oracle value
    depends on a rounding that sits on a bf16 midpoint (flagged from the oracle's
    pre-rounding values `pre` = (raw_pre, y_pre)); those may differ by <= MAX_FLIP_ULPS
    ulps and must stay rare.  A y counts as sensitive within the midpoint window widened by
    the rstd shift its row's sensitive raw elements can cause (rstd_shift_ulps).  The
    reference's own tolerance must hold everywhere."""
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    assert a.shape == e.shape, (a.shape, e.shape)
    assert torch.isfinite(a).all(), f"{label}: non-finite values"
    diff = (a - e).abs()
    bad = diff > atol + rtol * e.abs()
    excused = torch.zeros_like(bad)
    if bad.any():
        assert pre is not None, f"{label}: {int(bad.sum())} elements outside rtol/atol"
        raw_pre, y_pre = (t.detach().float().cpu() for t in pre)
        y_low16 = (y_pre.contiguous().view(torch.int32) & 0xFFFF).float() / 65536.0
        y_window = MIDPOINT_WINDOW + rstd_shift_ulps(raw_pre, y_pre)
        sensitive = near_bf16_midpoint(raw_pre) | ((y_low16 - 0.5).abs() < y_window)
        # ulp of the larger magnitude: a flip next to a power of two crosses into the
        # coarser binade (e.g. 0.99609375 vs 1.0078125)
        ulp = bf16_ulp(torch.maximum(a.abs(), e.abs()))
        excused = bad & sensitive & (diff <= MAX_FLIP_ULPS * ulp + atol)
        unexplained = bad & ~excused
        if unexplained.any():
            idx = unexplained.nonzero()[0].tolist()
            raise AssertionError(
                f"{label}: {int(unexplained.sum())} elements outside rtol={rtol}/atol={atol} "
                f"and not rounding-sensitive; first at {idx}: got {a[tuple(idx)].item()} "
                f"expected {e[tuple(idx)].item()}"
            )
        fraction = excused.float().mean().item()
        assert fraction <= MAX_FLIP_FRACTION, f"{label}: {fraction:.2e} rounding flips"
    torch.testing.assert_close(a, e, atol=REF_OUT_ATOL, rtol=REF_OUT_RTOL)
    return {"flips": int(excused.sum()), "elements": a.numel()}


def assert_states(actual: torch.Tensor, expected: torch.Tensor, *, rtol: float = RTOL,
                  atol: float = ATOL, label: str = "state") -> None:
    torch.testing.assert_close(actual.detach().cpu(), expected.detach().cpu(), rtol=rtol,
                               atol=atol, msg=lambda m: f"{label}: {m}")
