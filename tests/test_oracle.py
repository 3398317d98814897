"""Pins the CPU oracle (oracle/gdn.py, oracle/brute.py) before the parity tests rely on it:
golden vectors written by the reference's own post_conv_gdn, the reference's closed-form
scalar recurrence, an fp64 brute force, delta-rule invariants, transformers' independent
Qwen3-Next statement of the recurrence, and planted mistakes that each of those checks must
catch."""

from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from oracle import brute, gdn

FIELDS = ("q", "k", "v", "a", "b", "a_log", "dt_bias", "gate", "norm_weight")


def run_golden(d, **kw):
    eps = float(d["eps"]) if "eps" in d else 1e-6
    return gdn.run(*(d[f] for f in FIELDS), d["state"], d["lengths"], norm_eps=eps, **kw)


@pytest.mark.parametrize("name", ["scalar", "prefix", "tiny_bf16", "cfg1_step", "mtp"])
def test_oracle_reproduces_reference_vectors(golden, name):
    d = golden(name)
    out, final, ckpt = run_golden(d, save_checkpoints="checkpoints" in d)
    # Same op sequence and rounding points as the reference: bit-identical on one machine.
    assert out.dtype == d["output"].dtype
    assert torch.equal(out, d["output"])
    assert torch.equal(final, d["final_state"])
    if "checkpoints" in d:
        assert torch.equal(ckpt, d["checkpoints"])


def test_oracle_reproduces_reference_64_steps(golden):
    d = golden("cfg1_64")
    state = d["state"]
    outs = []
    for t in range(64):
        step = [d[f][:, t:t + 1] for f in ("q", "k", "v", "a", "b")]
        o, state, _ = gdn.run(*step, d["a_log"], d["dt_bias"], d["gate"][:, t:t + 1],
                              d["norm_weight"], state, d["lengths"])
        outs.append(o)
    assert torch.equal(torch.cat(outs, 1), d["output"])
    assert torch.equal(state, d["final_state"])


def test_scalar_closed_form():
    """Reference tests/test_gdn.py:47-55: decay 1/2 and beta 1/2 from zero projections,
    S1 = 1 + 0.5*(3 - kappa)*kappa with kappa = (1 + 1e-6)^-1/2."""
    one = torch.ones(1, 1, 1, 1)
    zero = torch.zeros(1, 1, 1)
    _, final, _ = gdn.run(one, one, one * 3, zero, zero, torch.zeros(1), torch.zeros(1), one,
                          torch.ones(1), one * 2, torch.ones(1, dtype=torch.int32))
    kappa = (1 + 1e-6) ** -0.5
    torch.testing.assert_close(final, one * (1 + 0.5 * (3 - kappa) * kappa))


def tiny_case(seed, batch=2, tokens=3, hk=1, hv=2, k=4, v=3, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    return dict(q=r(batch, tokens, hk, k).to(dtype), k=r(batch, tokens, hk, k).to(dtype),
                v=r(batch, tokens, hv, v).to(dtype), a=r(batch, tokens, hv).to(dtype),
                b=r(batch, tokens, hv).to(dtype), a_log=r(hv), dt_bias=r(hv),
                gate=r(batch, tokens, hv, v).to(dtype), norm_weight=r(v),
                state=r(batch, hv, v, k) * 0.5,
                lengths=torch.tensor([tokens, 1][:batch] + [0] * max(0, batch - 2)))


@pytest.mark.parametrize("seed,k,v", [(0, 5, 6), (1, 6, 5), (2, 5, 5), (3, 8, 8)])
def test_oracle_matches_fp64_brute_force(seed, k, v):
    c = tiny_case(seed, batch=3, tokens=4, hk=2, hv=4, k=k, v=v)
    c["lengths"] = torch.tensor([4, 2, 0])
    out, final, ckpt = gdn.run(*(c[f] for f in FIELDS), c["state"], c["lengths"],
                               save_checkpoints=True)
    np_in = [c[f].double().numpy() for f in FIELDS]
    b_out, b_final, b_states = brute.run(*np_in, c["state"].double().numpy(),
                                         c["lengths"].numpy(), round_raw=False)
    np.testing.assert_allclose(final.double().numpy(), b_final, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ckpt.double().numpy(), b_states, rtol=1e-5, atol=1e-6)
    # fp32 inputs: the oracle's `raw` rounding is to fp32, so compare unrounded brute output
    np.testing.assert_allclose(out.double().numpy(), b_out, rtol=1e-4, atol=1e-5)


def test_oracle_matches_brute_force_bf16_rounding():
    """bf16 inputs: the brute force's explicit bf16 rounding of `raw` and of the output."""
    c = tiny_case(11, batch=2, tokens=3, hk=1, hv=2, k=8, v=8, dtype=torch.bfloat16)
    out, _, _, (raw_pre, y_pre) = gdn.run(*(c[f] for f in FIELDS), c["state"], c["lengths"],
                                          return_pre=True)
    np_in = [c[f].float().double().numpy() for f in FIELDS]
    b_out, _, _ = brute.run(*np_in, c["state"].double().numpy(), c["lengths"].numpy())
    b_rounded = np.vectorize(brute.bf16_round)(b_out)
    got = out.float().double().numpy()
    # identical except where an fp32-vs-fp64 difference straddles a bf16 midpoint
    from tests.parity import near_bf16_midpoint

    sensitive = (near_bf16_midpoint(raw_pre, 0.01) | near_bf16_midpoint(y_pre, 0.01)).numpy()
    assert np.array_equal(got[~sensitive], b_rounded[~sensitive])


def test_prefix_invariant_and_padding():
    """T single-token calls equal one T-token call; inputs are not mutated; a length-0 row
    keeps its state bit-exactly and outputs zeros (reference tests/test_gdn.py:7-44)."""
    c = tiny_case(7, batch=3, tokens=4, hk=2, hv=6, k=5, v=7)
    c["lengths"] = torch.tensor([4, 2, 0])
    original = c["state"].clone()
    full = gdn.run(*(c[f] for f in FIELDS), c["state"], c["lengths"], save_checkpoints=True)
    running = c["state"]
    for t in range(4):
        step = [c[f][:, t:t + 1] if f in ("q", "k", "v", "a", "b", "gate") else c[f]
                for f in FIELDS]
        out, running, _ = gdn.run(*step, running, (c["lengths"] > t).int())
        torch.testing.assert_close(out[:, 0], full[0][:, t])
        torch.testing.assert_close(running, full[2][:, t + 1])
    assert torch.equal(c["state"], original)
    assert torch.equal(full[1][2], original[2])
    assert full[0][2].count_nonzero() == 0


def test_identity_when_decay_one_and_beta_zero():
    c = tiny_case(3)
    c["a_log"] = torch.full_like(c["a_log"], -math.inf)  # exp(A_log) = 0 -> decay = 1
    c["b"] = torch.full_like(c["b"], -math.inf)  # sigmoid(-inf) = 0 -> beta = 0
    c["lengths"] = torch.tensor([3, 3])
    _, final, _ = gdn.run(*(c[f] for f in FIELDS), c["state"], c["lengths"])
    assert torch.equal(final, c["state"])


def test_beta_one_projects_onto_v():
    """beta = 1: after the update S' k^ = v up to |k^|^2 = |k|^2/(|k|^2+1e-6) (delta rule)."""
    c = tiny_case(5, batch=1, tokens=1, hk=1, hv=1, k=16, v=8)
    c["b"] = torch.full_like(c["b"], math.inf)
    _, final, _ = gdn.run(*(c[f] for f in FIELDS), c["state"], torch.tensor([1]))
    k = c["k"][0, 0, 0].double()
    k_hat = k / torch.sqrt(k.square().sum() + 1e-6)
    proj = final[0, 0].double() @ k_hat
    torch.testing.assert_close(proj, c["v"][0, 0, 0].double(), rtol=1e-5, atol=1e-5)


def test_q_unit_vector_reads_state_column():
    """q = e_j selects column j of S (the K axis is the contracted one)."""
    c = tiny_case(9, batch=1, tokens=1, hk=1, hv=1, k=6, v=5)
    c["q"] = torch.zeros_like(c["q"])
    c["q"][..., 2] = 1.0
    c["gate"] = torch.full_like(c["gate"], 30.0)  # silu(30) = 30 (to fp32)
    c["norm_weight"] = torch.ones_like(c["norm_weight"])
    out, final, _, (raw_pre, _) = gdn.run(*(c[f] for f in FIELDS), c["state"], torch.tensor([1]),
                                          return_pre=True)
    scale = (1 + 1e-6) ** -0.5 * 6**-0.5
    torch.testing.assert_close(raw_pre[0, 0, 0], final[0, 0, :, 2] * scale, rtol=1e-6, atol=0)


# ---- planted mistakes: each must be caught by one of the checks above ------------------------


def _run_with(monkeypatch, name, fn, check):
    monkeypatch.setattr(gdn, name, fn)
    with pytest.raises(AssertionError):
        check()


def test_planted_mistakes_are_caught(monkeypatch, golden):
    original_recur, original_emit = gdn.recur, gdn.emit

    def decay_after_prediction(state, k_t, v_t, decay_t, beta_t, live):
        pred = (state * k_t[:, :, None, :]).sum(-1)
        delta = (v_t - pred) * beta_t[..., None]
        updated = state * decay_t[..., None, None] + delta[..., None] * k_t[:, :, None, :]
        return torch.where(live[:, None, None, None], updated, state)

    def transposed_state(state, k_t, v_t, decay_t, beta_t, live):
        return original_recur(state.transpose(-1, -2), k_t, v_t, decay_t, beta_t, live
                              ).transpose(-1, -2)

    def no_raw_rounding(state, q_t, gate_t, norm_weight, live, dtype, eps):
        raw = (state * q_t[:, :, None, :]).sum(-1)
        y = raw * torch.rsqrt(raw.square().mean(-1, keepdim=True) + eps)
        y = y * norm_weight.float() * torch.nn.functional.silu(gate_t.float())
        y = torch.where(live[:, None, None], y, 0)
        return y.to(dtype), raw, y

    def golden_check():
        d = golden("cfg1_step")
        out, final, _ = run_golden(d)
        assert torch.equal(out, d["output"]) and torch.equal(final, d["final_state"])

    def brute_check():
        test_oracle_matches_fp64_brute_force(2, 5, 5)

    for planted in (decay_after_prediction, transposed_state):
        _run_with(monkeypatch, "recur", planted, golden_check)
        _run_with(monkeypatch, "recur", planted, brute_check)
        monkeypatch.setattr(gdn, "recur", original_recur)
    _run_with(monkeypatch, "emit", no_raw_rounding, golden_check)
    monkeypatch.setattr(gdn, "emit", original_emit)


def transformers_recurrence():
    os.environ.setdefault("HF_HUB_OFFLINE", "1")   # the module import needs no network
    os.environ.setdefault("TRANSFORMERS_OFFLINE", "1")
    module = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    return module.torch_recurrent_gated_delta_rule


def agrees_with_transformers_recurrence(run_fn, seed=31):
    """Whether `run_fn` (oracle.gdn.run's signature) gives, over 16 tokens at 2 qk / 4 v
    heads, the final state and pre-rounding outputs of transformers' Qwen3-Next
    torch_recurrent_gated_delta_rule (an independent fp32 statement of the gated delta
    rule: state [K, V], l2-normalised q and k, q scaled by K^-1/2, g the log-decay) to
    rtol 1e-4 / atol 1e-5 (the two sum in different orders)."""
    rule = transformers_recurrence()
    g = torch.Generator().manual_seed(seed)
    batch, tokens, heads, v_heads, dim = 2, 16, 2, 4, 32
    q = torch.randn(batch, tokens, heads, dim, generator=g).bfloat16()
    k = torch.randn(batch, tokens, heads, dim, generator=g).bfloat16()
    v = torch.randn(batch, tokens, v_heads, dim, generator=g).bfloat16()
    a = torch.randn(batch, tokens, v_heads, generator=g).bfloat16()
    b = torch.randn(batch, tokens, v_heads, generator=g).bfloat16()
    a_log = torch.rand(v_heads, generator=g) * 2 - 1
    dt_bias = torch.randn(v_heads, generator=g)
    gate = torch.randn(batch, tokens, v_heads, dim, generator=g).bfloat16()
    weight = torch.randn(dim, generator=g)
    state0 = torch.randn(batch, v_heads, dim, dim, generator=g) * 0.02   # [B, Hv, V, K]
    lengths = torch.full((batch,), tokens)
    _, state, _, (raw_pre, _) = run_fn(q, k, v, a, b, a_log, dt_bias, gate, weight, state0,
                                       lengths, return_pre=True)
    group = v_heads // heads
    log_decay = -a_log.exp() * torch.nn.functional.softplus(a.float() + dt_bias)
    out, final = rule(q.float().repeat_interleave(group, 2), k.float().repeat_interleave(group, 2),
                      v.float(), log_decay, b.float().sigmoid(), state0.transpose(-1, -2).clone(),
                      True, use_qk_l2norm_in_kernel=True)
    return (torch.allclose(state, final.transpose(-1, -2), rtol=1e-4, atol=1e-5)
            and torch.allclose(raw_pre, out, rtol=1e-4, atol=1e-5))


def test_oracle_matches_transformers_recurrence():
    """The recurrence and its raw outputs agree with transformers' independent statement."""
    assert agrees_with_transformers_recurrence(gdn.run)


def test_transformers_recurrence_check_catches_late_decay(monkeypatch):
    """A planted mistake -- the prediction taken from the state before the decay -- fails
    the check above."""
    transformers_recurrence()

    def late_decay(state, k_t, v_t, decay_t, beta_t, live):
        pred = (state * k_t[:, :, None, :]).sum(-1)
        delta = (v_t - pred) * beta_t[..., None]
        updated = state * decay_t[..., None, None] + delta[..., None] * k_t[:, :, None, :]
        return torch.where(live[:, None, None, None], updated, state)

    monkeypatch.setattr(gdn, "recur", late_decay)
    assert not agrees_with_transformers_recurrence(gdn.run)
