"""Causal depthwise conv1d update of one decode token -- test infrastructure.

The pre-GDN step of the decode layer (vLLM 0.29 `causal_conv1d_update`, called at the
reference's python/lightdelta/integration/vllm_layer.py:199-207; vLLM is a third-party
dependency absent here, so this restates its published algorithm for the single-token
decode case):

  window[d] = [state[d, L-W+1 .. L-1], x[d]]            (the last W-1 state columns, x)
  acc[d]    = bias[d]; acc[d] = fma(weight[d, j], window[d, j], acc[d]) for j = 0 .. W-1
  y[d]      = bf16( silu(acc[d]) )                      (fp32 accumulation, oldest tap first)
  state[d]  = [state[d, 1 .. L-1], x[d]]                (shift left by one, append x)

The fp32 fused multiply-add chain is emulated exactly in float64 (a product of two fp32
values is exact in float64 and the single rounding back to fp32 is that of an fma).  The
SiLU is evaluated in float64 and rounded once, to the nearest bf16 (ties to even): the
exact value's rounding.  Any fp32 SiLU rounds to the same bf16 except within a few fp32
ulps of a bf16 rounding midpoint, where implementations legitimately differ; fixing the
exact rounding makes the conv output a deterministic function of its inputs.

State layout `[D, L]` per slot (dim-first); a dim-last pool is passed transposed.

Parity of this function is pinned only definitionally (it is checked against
torch.nn.functional.conv1d with groups = D and against an element loop); no reference test
or fixture covers the conv, so conv parity is "unpinned" in the reference's sense.
"""

from __future__ import annotations

import numpy as np
import torch
from torch.nn import functional as F


def round_to_bf16(y: np.ndarray) -> torch.Tensor:
    """float64 values rounded once to the nearest bf16, ties to even (no double rounding
    through fp32: where the fp32 rounding lands exactly on a bf16 midpoint that the float64
    value is not on, the direction comes from the float64 value)."""
    t = y.astype(np.float32)
    u = t.view(np.uint32).astype(np.int64)
    rne = torch.from_numpy(t).to(torch.bfloat16).view(torch.int16).numpy().astype(np.int64) & 0xFFFF
    tie = ((u & 0xFFFF) == 0x8000) & (t.astype(np.float64) != y) & np.isfinite(y)
    away = (np.abs(y) > np.abs(t.astype(np.float64))).astype(np.int64)
    bits = np.where(tie, (u >> 16) + away, rne).astype(np.uint16)
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)


def conv_update(x: torch.Tensor, state: torch.Tensor, weight: torch.Tensor, bias=None):
    """x [B, D] (bf16); state [B, D, L]; weight [D, W]; bias [D] or None.
    Returns (y [B, D] bf16, new_state [B, D, L] in state's dtype)."""
    width = weight.shape[1]
    window = torch.cat([state[..., state.shape[-1] - (width - 1):], x[..., None]], -1).float()
    acc = torch.zeros(window.shape[:-1], dtype=torch.float32)
    if bias is not None:
        acc = acc + bias.float()
    for j in range(width):
        acc = (window[..., j].double() * weight[:, j].float().double() + acc.double()).float()
    a = acc.double().numpy()
    with np.errstate(over="ignore"):
        y = round_to_bf16(a / (1.0 + np.exp(-a)))
    new_state = torch.cat([state[..., 1:], x[..., None].to(state.dtype)], -1)
    return y, new_state


def conv_update_reference_form(x, state, weight, bias=None):
    """The same output through torch.nn.functional.conv1d (depthwise, groups = D)."""
    width = weight.shape[1]
    window = torch.cat([state[..., state.shape[-1] - (width - 1):], x[..., None]], -1).float()
    out = F.conv1d(window, weight.float()[:, None, :], bias=None if bias is None else bias.float(),
                   groups=weight.shape[0])
    return F.silu(out[..., 0]).to(x.dtype)
