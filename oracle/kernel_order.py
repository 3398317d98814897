"""The reference CUDA kernel's arithmetic order, restated on the CPU -- test infrastructure.

Only tests/ import this.  It answers one question: how often does a correct kernel whose
fp32 sums run in another order than Torch's land on the other side of a bf16 rounding?
It runs the recurrence and the gated RMSNorm of the reference's
`gdn_decode_post_conv_mtp_kernel` (csrc/gdn_decode.cu:230-353) in that kernel's order on
the oracle's prepared inputs (oracle.gdn.prepare: the same q^, k^, decay and beta) and with
the oracle's elementwise functions (rsqrt, silu), so that the summation order and the
contraction of multiply-adds are the only differences from oracle.gdn:

  * a row's dot products (S k^ and S q^, csrc/gdn_decode.cu:263-287): lane l of a 32-lane
    warp holds k = 4l .. 4l+3 and accumulates h[i] * x[i] for i = 0..3 from 0 as fused
    multiply-adds (nvcc contracts `acc += a * b`), then the warp sums the lanes by an xor
    butterfly over offsets 16, 8, 4, 2, 1 (warp_reduce_sum_pair, :109-118);
  * decay first (h *= decay, :266), delta = (v - S k^) * beta (:281-283), the update
    h += k^ * delta as a fused multiply-add (:286);
  * raw = bf16(S q^) (:292-299);
  * the norm's sum of squares (:325-333): lane l holds raw[l + 32 i], i = 0..3, summed as
    fused multiply-adds from 0, then the xor butterfly; rstd = rsqrt(ss / 128 + eps); the
    output ((raw * rstd) * w) * silu(gate) rounded to bf16 (:334-350).

Fused multiply-adds are formed in float64 and rounded once to float32: the product of two
float32 values is exact in float64, and the float64 sum rounds to float32 correctly except
when its own rounding lands on a float32 midpoint (probability about 2^-29 per operation).

Pinned by tests/test_kernel_order_cpu.py: the lane dot and the butterfly against exact
integer sums, a planted mistake (a butterfly with a missing stage) caught, and agreement
with oracle.gdn within the reference's own tolerance over many steps.
"""

from __future__ import annotations

import torch
from torch.nn import functional as F

from . import gdn

LANES = 32
PER_LANE = 4
BUTTERFLY = (16, 8, 4, 2, 1)


def fma32(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
    """fp32 a * b + c with one rounding (formed in float64)."""
    return (a.double() * b.double() + c.double()).float()


def lane_sum(partial: torch.Tensor, offsets=BUTTERFLY) -> torch.Tensor:
    """The xor butterfly over the last axis (32 lanes): every lane adds its partner's value,
    offset by offset; returns lane 0's total (every lane holds the same bits, as addition
    commutes)."""
    lanes = torch.arange(LANES)
    for off in offsets:
        partial = partial + partial[..., lanes ^ off]
    return partial[..., 0]


def lane_dot(h: torch.Tensor, x: torch.Tensor, offsets=BUTTERFLY) -> torch.Tensor:
    """sum_k h[..., k] x[..., k] over the last axis (128) in the kernel's order: per lane a
    fused multiply-add chain over its 4 consecutive k from 0, then the lane butterfly."""
    hl = h.reshape(*h.shape[:-1], LANES, PER_LANE)
    xl = x.expand_as(h).reshape(*h.shape[:-1], LANES, PER_LANE)
    acc = torch.zeros(hl.shape[:-1], dtype=torch.float32)
    for i in range(PER_LANE):
        acc = fma32(hl[..., i], xl[..., i], acc)
    return lane_sum(acc, offsets)


def step(state, k_t, v_t, decay_t, beta_t, q_t, gate_t, norm_weight, eps, offsets=BUTTERFLY):
    """One token for every (row, head): state [B, Hv, V, K] fp32; k_t, q_t [B, Hv, K];
    v_t [B, Hv, V]; decay_t, beta_t [B, Hv]; gate_t [B, Hv, V] (bf16).  Returns
    (new state, bf16 output [B, Hv, V], raw [B, Hv, V] as bf16 values in fp32)."""
    h = state * decay_t[..., None, None]
    pred = lane_dot(h, k_t[:, :, None, :], offsets)
    delta = (v_t - pred) * beta_t[..., None]
    h = fma32(k_t[:, :, None, :].expand_as(h), delta[..., None].expand_as(h), h)
    raw = lane_dot(h, q_t[:, :, None, :], offsets).to(torch.bfloat16).float()
    # lane l of the epilogue holds raw[l + 32 i]
    lanes = raw.reshape(*raw.shape[:-1], PER_LANE, LANES)
    ss = torch.zeros(lanes.shape[:-2] + (LANES,), dtype=torch.float32)
    for i in range(PER_LANE):
        ss = fma32(lanes[..., i, :], lanes[..., i, :], ss)
    ss = lane_sum(ss, offsets)
    rstd = torch.rsqrt(ss / 128.0 + eps)
    y = raw * rstd[..., None] * norm_weight.float() * F.silu(gate_t.float())
    return h, y.to(torch.bfloat16), raw


def run_steps(q, k, v, a, b, a_log, dt_bias, gate, norm_weight, initial_state, eps=1e-6,
              offsets=BUTTERFLY):
    """T in-place tokens on every row from initial_state [B, Hv, V, K]; inputs as
    oracle.gdn.run's ([B, T, ...]).  Returns (outputs [B, T, Hv, V] bf16, final state)."""
    p = gdn.prepare(q, k, v, a, b, a_log, dt_bias)
    state = initial_state.float()
    outs = []
    for t in range(q.shape[1]):
        state, out, _ = step(state, p.k[:, t], p.v[:, t], p.decay[:, t], p.beta[:, t],
                             p.q[:, t], gate[:, t], norm_weight, eps, offsets)
        outs.append(out)
    return torch.stack(outs, 1), state
