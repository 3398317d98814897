"""Pins the conv oracle (oracle/conv.py): against torch.nn.functional.conv1d with groups =
channels, an element loop and planted mistakes, the multi-token form against repeated
single-token updates, and the standard non-speculative layout (3 state columns, one token)
against transformers' independent Qwen3-Next statement of the update.  No reference test or
fixture covers the conv (it lives in vLLM), so vLLM's column convention for speculative
steps (num_accepted_tokens, longer states) stays unpinned beyond these checks."""

from __future__ import annotations

import math
import os

import numpy as np

import pytest
import torch

from oracle import conv


def case(seed, batch=3, channels=6, length=3, bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, channels, generator=g).bfloat16()
    state = torch.randn(batch, channels, length, generator=g).bfloat16()
    weight = (torch.randn(channels, 4, generator=g) / 2).bfloat16()
    b = torch.randn(channels, generator=g).bfloat16() if bias else None
    return x, state, weight, b


@pytest.mark.parametrize("length,bias", [(3, False), (3, True), (4, False), (6, True)])
def test_conv_matches_conv1d_groups(length, bias):
    x, state, weight, b = case(length, length=length, bias=bias)
    y, _ = conv.conv_update(x, state, weight, b)
    ref = conv.conv_update_reference_form(x, state, weight, b)
    # both round an fp32 sum of 4 products (+ bias) to bf16; summation order may differ
    torch.testing.assert_close(y.float(), ref.float(), rtol=8e-3, atol=1e-2)


def test_conv_element_loop_and_state_shift():
    x, state, weight, b = case(1, batch=2, channels=4, length=5)
    y, new_state = conv.conv_update(x, state, weight, b)
    for r in range(2):
        for d in range(4):
            window = [float(state[r, d, j]) for j in range(2, 5)] + [float(x[r, d])]
            acc = float(b[d]) + sum(float(weight[d, j]) * window[j] for j in range(4))
            expect = acc / (1 + math.exp(-acc))
            assert abs(float(y[r, d]) - expect) <= 0.008 * abs(expect) + 1e-3
            assert [float(v) for v in new_state[r, d]] == [float(state[r, d, j]) for j in range(1, 5)] + [float(x[r, d])]


def loop_check(x, state, weight, b, y):
    """The element-loop statement of the conv, as a pass/fail predicate."""
    length = state.shape[-1]
    for r in range(x.shape[0]):
        for d in range(x.shape[1]):
            window = [float(state[r, d, j]) for j in range(length - 3, length)] + [float(x[r, d])]
            acc = (float(b[d]) if b is not None else 0.0) + sum(
                float(weight[d, j]) * window[j] for j in range(4))
            expect = acc / (1 + math.exp(-acc))
            if abs(float(y[r, d]) - expect) > 0.008 * abs(expect) + 1e-3:
                return False
    return True


@pytest.mark.parametrize("mistake", ["reversed_taps", "oldest_window", "dropped_bias", "no_silu"])
def test_planted_conv_mistakes_fail_the_loop_check(mistake):
    x, state, weight, b = case(7, batch=2, channels=8, length=4)
    assert loop_check(x, state, weight, b, conv.conv_update(x, state, weight, b)[0])
    if mistake == "reversed_taps":
        y = conv.conv_update(x, state, weight.flip(1), b)[0]
    elif mistake == "oldest_window":  # window from the first state columns instead of the last
        y = conv.conv_update(x, torch.cat([state[..., :3], state[..., :1]], -1), weight, b)[0]
    elif mistake == "dropped_bias":
        y = conv.conv_update(x, state, weight, None)[0]
    else:
        window = torch.cat([state[..., 1:], x[..., None]], -1).float()
        y = ((window * weight.float()).sum(-1) + b.float()).bfloat16()
    assert not loop_check(x, state, weight, b, y)


def test_fma_chain_and_correct_rounding():
    """The oracle's conv output is the float64 SiLU of an fp32 fma chain (one rounding per
    tap, oldest first), rounded once to the nearest bf16."""
    x, state, weight, b = case(3, batch=2, channels=5, length=3)
    y, _ = conv.conv_update(x, state, weight, b)
    for r in range(2):
        for d in range(5):
            window = [float(state[r, d, j]) for j in range(3)] + [float(x[r, d])]
            acc = np.float32(float(b[d]))
            for j in range(4):
                acc = np.float32(np.float64(weight[d, j].item()) * window[j] + np.float64(acc))
            exact = float(acc) / (1 + math.exp(-float(acc)))
            assert float(y[r, d]) == float(nearest_bf16(exact))


def nearest_bf16(v: float) -> float:
    """Brute force: the bf16 nearest to v (ties to the even significand)."""
    t = torch.tensor([v], dtype=torch.float64).float()
    bits = int(t.view(torch.int32)) & 0xFFFFFFFF
    lo = torch.tensor([(bits >> 16) << 16], dtype=torch.int64).to(torch.int32).view(torch.float32)
    hi = torch.tensor([((bits >> 16) + 1) << 16], dtype=torch.int64).to(torch.int32).view(
        torch.float32)
    lo, hi = float(lo), float(hi)
    dl, dh = abs(v - lo), abs(v - hi)
    if dl != dh:
        return lo if dl < dh else hi
    return lo if ((bits >> 16) & 1) == 0 else hi


def test_round_to_bf16_is_single_rounding():
    """Against brute force, on values whose fp32 rounding lands exactly on a bf16 midpoint
    (where rounding through fp32 would round twice) and on random values."""
    rng = np.random.default_rng(0)
    mids = (rng.integers(0x3C00, 0x4200, 200).astype(np.uint32) << 16) | 0x8000
    mid_vals = mids.view(np.float32).astype(np.float64)
    # nudge off the midpoint by less than half an fp32 ulp: fp32 rounds back onto it
    nudged = mid_vals * (1 + rng.choice([-1.0, 1.0], 200) * rng.uniform(1e-9, 2.5e-8, 200))
    assert (nudged.astype(np.float32) == mid_vals.astype(np.float32)).all()
    through_fp32 = torch.from_numpy(nudged.astype(np.float32)).to(torch.bfloat16).float()
    values = np.concatenate([nudged, mid_vals, rng.normal(0, 3, 300)])
    got = conv.round_to_bf16(values).float().numpy()
    want = np.array([nearest_bf16(float(v)) for v in values])
    np.testing.assert_array_equal(got, want)
    # the double rounding the oracle avoids would disagree on some of the nudged values
    assert (through_fp32.numpy() != got[:200]).any()


def spec_case(seed, channels=5, cols=6, length=4):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(length, channels, generator=g).bfloat16()
    state = torch.randn(channels, cols, generator=g).bfloat16()
    weight = (torch.randn(channels, 4, generator=g) / 2).bfloat16()
    bias = torch.randn(channels, generator=g).bfloat16()
    return x, state, weight, bias


def test_single_token_step_is_the_plain_update():
    x, state, weight, bias = spec_case(1, cols=3, length=1)
    y, new_state = conv.conv_update_tokens(x, state, weight, bias, offset=0)
    y1, new1 = conv.conv_update(x, state[None], weight, bias)
    assert torch.equal(y, y1) and torch.equal(new_state, new1[0])


@pytest.mark.parametrize("offset", [0, 1, 2, 3])
def test_multi_token_outputs_equal_a_rolling_single_token_conv(offset):
    """Token t's output is the single-token update applied after tokens 0..t-1, starting
    from the W-1 history columns at the offset."""
    x, state, weight, bias = spec_case(2 + offset)
    y, _ = conv.conv_update_tokens(x, state, weight, bias, offset=offset)
    rolling = state[None, :, offset:offset + 3]
    for t in range(x.shape[0]):
        yt, rolling = conv.conv_update(x[t][None], rolling, weight, bias)
        assert torch.equal(y[t], yt[0])


@pytest.mark.parametrize("offset", [0, 1, 2, 3])
def test_next_step_history_ends_at_each_accepted_token(offset):
    """The defining property of the speculative conv state: after a step with L tokens,
    accepting n of them (the next step's offset n-1) selects the W-1 inputs that end at
    x_{n-1} in the sequence history ++ x.  A plain shift by L (the non-speculative update)
    violates it."""
    x, state, weight, bias = spec_case(10 + offset)
    length = x.shape[0]
    _, new_state = conv.conv_update_tokens(x, state, weight, bias, offset=offset)
    seq = torch.cat([state[:, offset:offset + 3], x.t()], -1)
    for n in range(1, length + 1):
        assert torch.equal(new_state[:, n - 1:n + 2], seq[:, n:n + 3])
    if offset != length - 1:  # where a plain shift by L coincides with the update
        shifted = torch.cat([state[:, length:], x.t()], -1)  # planted mistake
        assert not all(torch.equal(shifted[:, n - 1:n + 2], seq[:, n:n + 3])
                       for n in range(1, length + 1))



def transformers_update():
    os.environ.setdefault("HF_HUB_OFFLINE", "1")   # the module import needs no network
    os.environ.setdefault("TRANSFORMERS_OFFLINE", "1")
    module = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    return getattr(module.causal_conv1d_update, "__wrapped__", module.causal_conv1d_update)


def agrees_with_transformers(update_tokens, seed):
    """Whether `update_tokens` (conv_update_tokens' signature) matches transformers'
    statement of the standard layout on random requests: the same new state bit for bit,
    and outputs that are the bf16 rounding of its fp32 conv (within the fp32 error of two
    summation orders)."""
    update = transformers_update()
    g = torch.Generator().manual_seed(seed)
    batch, channels = 4, 64
    for bias in (False, True):
        x = torch.randn(batch, channels, generator=g).bfloat16()
        state = torch.randn(batch, channels, 3, generator=g).bfloat16()
        weight = (torch.randn(channels, 4, generator=g) / 2).bfloat16()
        b = torch.randn(channels, generator=g).bfloat16() if bias else None
        hf_state = state.float().clone()
        hf_out = update(x.float()[:, :, None], hf_state, weight.float(),
                        None if b is None else b.float(), "silu")[:, :, 0]
        for r in range(batch):
            y, new_state = update_tokens(x[r:r + 1], state[r], weight, b, offset=0)
            if not torch.equal(new_state.float(), hf_state[r]):
                return False
            got, ref = y[0].float(), hf_out[r]
            ulp = 2.0 ** (torch.floor(torch.log2(ref.abs().clamp_min(2.0**-126))) - 7)
            if not ((got - ref).abs() <= 0.5 * ulp + 1e-5 * ref.abs() + 1e-30).all():
                return False
    return True


def test_standard_layout_matches_transformers_conv_update():
    """The standard non-speculative layout (a conv state of width - 1 = 3 columns, one token,
    no accepted offset) is where vLLM's update and the causal_conv1d semantics coincide:
    append the token, keep the last 3 columns, convolve the 4-column window, SiLU.
    transformers' Qwen3-Next layer carries a pure-torch statement of that update
    (modeling_qwen3_next.causal_conv1d_update, its fallback when no fused kernel is
    installed), an implementation independent of this oracle, which must agree with it."""
    assert agrees_with_transformers(conv.conv_update_tokens, seed=11)


def test_transformers_check_catches_a_conv_after_the_shift():
    """A planted mistake -- convolving the shifted state (history [s1, s2, x]) instead of the
    state before the token -- fails the transformers check."""
    transformers_update()

    def shifted_first(x, state, weight, bias=None, offset=0):
        _, new_state = conv.conv_update_tokens(x, state, weight, bias, offset)
        y, _ = conv.conv_update(x, new_state[None], weight, bias)
        return y, new_state

    assert not agrees_with_transformers(shifted_first, seed=12)
