"""fp32 CPU restatement of the reference's unfused post-conv GDN -- test infrastructure.

Follows python/lightdelta/reference/gdn.py:97-128 stage by stage, keeping its rounding
points (each torch op rounds to fp32; `raw` is rounded to the input dtype before the norm;
the output is cast to the input dtype):

  prepare()   gdn.py:97-105   q,k L2 norm (+1e-6), GQA head expansion, q * K^-1/2,
                              decay = exp(-exp(A_log) * softplus(a + dt_bias)), beta = sigmoid(b)
  recur()     gdn.py:110-115  decayed = S*decay; pred = sum_K(decayed*k);
                              delta = (v - pred)*beta; S' = decayed + delta*k; masked by live
  emit()      gdn.py:116-120  raw = dtype(sum_K(S*q)); raw*rsqrt(mean(raw^2)+eps)*w*silu(gate),
                              zero where not live, cast to dtype
  run()       gdn.py:70-128   T tokens, optional per-token checkpoints (index 0 = initial)

Pinned by: tests/golden/*.npz written by the reference's own post_conv_gdn (bit-level
agreement is checked), the closed form of tests/test_gdn.py:47-55, the fp64 brute force in
oracle/brute.py, and the delta-rule invariants in tests/test_oracle.py.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch.nn import functional as F


@dataclass
class Prepared:
    q: torch.Tensor  # [B, T, Hv, K] fp32, normalised and scaled
    k: torch.Tensor  # [B, T, Hv, K] fp32, normalised
    v: torch.Tensor  # [B, T, Hv, V] fp32
    decay: torch.Tensor  # [B, T, Hv] fp32
    beta: torch.Tensor  # [B, T, Hv] fp32


def l2_normalize(x: torch.Tensor) -> torch.Tensor:
    """x * rsqrt(sum(x^2) + 1e-6) over the last axis (reference gdn.py:98-99)."""
    return x * torch.rsqrt(x.square().sum(-1, keepdim=True) + 1e-6)


def prepare(q, k, v, a, b, a_log, dt_bias) -> Prepared:
    key_heads, key_dim = q.shape[-2:]
    group = v.shape[-2] // key_heads
    qn = l2_normalize(q.float()).repeat_interleave(group, dim=2) * key_dim**-0.5
    kn = l2_normalize(k.float()).repeat_interleave(group, dim=2)
    g = -a_log.exp() * F.softplus(a.float() + dt_bias.float())
    return Prepared(qn, kn, v.float(), g.exp(), b.float().sigmoid())


def recur(state, k_t, v_t, decay_t, beta_t, live):
    """One masked delta-rule update.  state [B,Hv,V,K]; k_t [B,Hv,K]; v_t [B,Hv,V];
    decay_t, beta_t [B,Hv]; live [B] bool."""
    decayed = state * decay_t[..., None, None]
    pred = (decayed * k_t[:, :, None, :]).sum(-1)
    delta = (v_t - pred) * beta_t[..., None]
    updated = decayed + delta[..., None] * k_t[:, :, None, :]
    return torch.where(live[:, None, None, None], updated, state)


def emit(state, q_t, gate_t, norm_weight, live, dtype, eps):
    """Rounded recurrence output through the gated RMSNorm.  q_t [B,Hv,K]; gate_t [B,Hv,V].
    Returns (output in dtype, raw before its rounding, y before the final cast), the last
    two in fp32 -- the values whose rounding decides each output element."""
    raw_pre = (state * q_t[:, :, None, :]).sum(-1)
    raw = raw_pre.to(dtype).float()
    y = raw * torch.rsqrt(raw.square().mean(-1, keepdim=True) + eps)
    y = y * norm_weight.float() * F.silu(gate_t.float())
    y = torch.where(live[:, None, None], y, 0)
    return y.to(dtype), raw_pre, y


def run(q, k, v, a, b, a_log, dt_bias, gate, norm_weight, initial_state, lengths,
        *, save_checkpoints=False, norm_eps=1e-6, return_pre=False):
    """T tokens for B rows.  Returns (output [B,T,Hv,V] dtype, final_state fp32,
    checkpoints [B,T+1,...] or [B,0,...]) and, with return_pre, a 4th element
    (raw_pre, y_pre): the fp32 values [B,T,Hv,V] rounded at the two rounding points."""
    p = prepare(q, k, v, a, b, a_log, dt_bias)
    dtype = q.dtype
    batch, tokens = q.shape[:2]
    state = initial_state
    outs, raws, ys = [], [], []
    history = [initial_state] if save_checkpoints else []
    for t in range(tokens):
        live = lengths > t
        state = recur(state, p.k[:, t], p.v[:, t], p.decay[:, t], p.beta[:, t], live)
        out_t, raw_t, y_t = emit(state, p.q[:, t], gate[:, t], norm_weight, live, dtype,
                                 norm_eps)
        outs.append(out_t)
        raws.append(raw_t)
        ys.append(y_t)
        if save_checkpoints:
            history.append(state)
    if save_checkpoints:
        checkpoints = torch.stack(history, 1)
    else:
        checkpoints = initial_state.new_empty((batch, 0, *initial_state.shape[1:]))
    result = (torch.stack(outs, 1), state, checkpoints)
    if return_pre:
        return result + ((torch.stack(raws, 1), torch.stack(ys, 1)),)
    return result
