"""The bf16 output comparison (tests/parity.py) on constructed cases: a raw value on a bf16
midpoint may round either way, and through the row's rstd that moves every y of the row;
a genuine error of one ulp elsewhere must still be caught."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from tests.parity import (MIDPOINT_WINDOW, assert_bf16_outputs, bf16_ulp, near_bf16_midpoint,
                          rstd_shift_ulps)


def cascade_case(seed: int, rows: int = 64, n: int = 128):
    """Rows of small raw outputs, exactly representable in bf16 except element 48 of row 0,
    which sits on a bf16 midpoint; the expected outputs round it one way, the actual ones
    the other way."""
    gen = torch.Generator().manual_seed(seed)
    raw_pre = (torch.randn(rows, n, generator=gen) * 0.006).bfloat16().float()
    low = raw_pre[0, 48]
    raw_pre[0, 48] = low + 0.5 * bf16_ulp(low) * torch.sign(low)
    gate = torch.randn(rows, n, generator=gen) * 2

    def finish(raw):
        y = raw * torch.rsqrt(raw.square().mean(-1, keepdim=True) + 1e-6)
        return y * F.silu(gate)

    raw_b = raw_pre.bfloat16().float()
    y_pre = finish(raw_b)
    raw_alt = raw_b.clone()
    raw_alt[0, 48] += bf16_ulp(raw_b[0, 48]) * torch.sign(raw_pre[0, 48] - raw_b[0, 48])
    return raw_pre, y_pre, y_pre.bfloat16(), finish(raw_alt).bfloat16()


def test_rstd_cascade_of_a_midpoint_raw_is_excused():
    raw_pre, y_pre, expected, actual = cascade_case(96)
    a, e = actual.float(), expected.float()
    bad = (a - e).abs() > 2e-3 + 2e-3 * e.abs()
    plain = near_bf16_midpoint(raw_pre) | near_bf16_midpoint(y_pre)
    assert (bad & ~plain).any(), "the case must contain a flip the plain window misses"
    stats = assert_bf16_outputs(actual, expected, (raw_pre, y_pre))
    assert stats["flips"] == int(bad.sum())


def test_rstd_shift_is_zero_without_sensitive_raw():
    raw_pre, y_pre, _, _ = cascade_case(96)
    raw_pre[0, 48] = raw_pre[0, 48].bfloat16().float()  # exactly representable: no ambiguity
    assert not near_bf16_midpoint(raw_pre).any()
    assert torch.equal(rstd_shift_ulps(raw_pre, y_pre), torch.zeros_like(y_pre))


def test_rstd_shift_matches_the_actual_change():
    raw_pre, y_pre, _, actual = cascade_case(96)
    shift = rstd_shift_ulps(raw_pre, y_pre)
    # y recomputed in fp32 with the other rounding moves by at most the bound (+ fp32 noise)
    raw_b = raw_pre.bfloat16().float()
    raw_alt = raw_b.clone()
    raw_alt[0, 48] += bf16_ulp(raw_b[0, 48]) * torch.sign(raw_pre[0, 48] - raw_b[0, 48])
    scale = torch.rsqrt(raw_alt.square().mean(-1, keepdim=True) + 1e-6) / torch.rsqrt(
        raw_b.square().mean(-1, keepdim=True) + 1e-6)
    moved = (y_pre * scale - y_pre).abs() / bf16_ulp(y_pre)
    mask = torch.arange(raw_pre.shape[-1]) != 48
    assert (moved[:, mask] <= shift[:, mask] * 1.001 + 1e-6).all()
    assert shift.max() > MIDPOINT_WINDOW  # the plain window alone would be too narrow


def test_genuine_one_ulp_error_is_caught():
    raw_pre, y_pre, expected, _ = cascade_case(96)
    raw_pre[0, 48] = raw_pre[0, 48].bfloat16().float()  # no sensitive raw anywhere
    y_pre = y_pre.clone()
    actual = y_pre.bfloat16()
    expected = actual.clone()
    # the largest y that is far from a midpoint, moved by one ulp
    far = ~near_bf16_midpoint(y_pre, 0.3)
    target = torch.where(far, y_pre.abs(), torch.zeros_like(y_pre)).argmax()
    flat = actual.view(-1)
    flat[target] = (flat[target].float() + bf16_ulp(flat[target].float())).bfloat16()
    with pytest.raises(AssertionError, match="not rounding-sensitive"):
        assert_bf16_outputs(actual, expected, (raw_pre, y_pre))
