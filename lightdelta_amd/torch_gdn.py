"""Unfused Torch GDN: the `compute = "torch_reference"` ablation of GDNBackend.

Public API of the reference module it stands in for (python/lightdelta/reference/gdn.py:15-128):
`GDNInputs`, `GDNResult`, `post_conv_gdn(inputs, initial_state, lengths, *,
save_checkpoints=False, norm_eps=1e-6)`.  It runs with plain torch ops on whatever device
its inputs live on; the backend uses it only when a config explicitly selects
`compute = "torch_reference"` (packed state, eager) -- it is never a fallback for the HIP
path, which raises when its library is missing.

Precision contract (reference gdn.py:97-120): q/k are L2-normalised in fp32, q scaled by
K^-1/2 after the GQA head expansion; the state is decayed before the prediction; the
recurrence output is rounded to the input dtype before the gated RMSNorm; the final output
is cast to the input dtype.  Rows whose `lengths` entry is <= t keep their state and get
zero output at token t.
"""

from __future__ import annotations

from dataclasses import dataclass, fields

import torch
from torch import Tensor
from torch.nn import functional as F


@dataclass(frozen=True)
class GDNInputs:
    q: Tensor  # [B, T, Hk, K] post-conv activations
    k: Tensor  # [B, T, Hk, K]
    v: Tensor  # [B, T, Hv, V]
    a: Tensor  # [B, T, Hv] raw decay projection
    b: Tensor  # [B, T, Hv] raw update projection
    a_log: Tensor  # [Hv] fp32
    dt_bias: Tensor  # [Hv]
    gate: Tensor  # [B, T, Hv, V] raw output gate
    norm_weight: Tensor  # [V]

    def validate(self) -> None:
        """Shape / dtype / device contract (reference gdn.py:27-60)."""
        if self.q.ndim != 4 or self.v.ndim != 4:
            raise ValueError("q and v must be [batch, tokens, heads, dimension]")
        batch, tokens, key_heads, key_dim = self.q.shape
        value_heads, value_dim = self.v.shape[-2:]
        if min(batch, tokens, key_heads, key_dim, value_heads, value_dim) <= 0:
            raise ValueError("Input dimensions must be positive; padding uses lengths=0")
        if value_heads % key_heads:
            raise ValueError("Value heads must be divisible by key heads")
        shapes = {
            "k": tuple(self.q.shape),
            "v": (batch, tokens, value_heads, value_dim),
            "a": (batch, tokens, value_heads),
            "b": (batch, tokens, value_heads),
            "a_log": (value_heads,),
            "dt_bias": (value_heads,),
            "gate": tuple(self.v.shape),
            "norm_weight": (value_dim,),
        }
        for name, shape in shapes.items():
            if tuple(getattr(self, name).shape) != shape:
                raise ValueError(f"{name} must have shape {shape}")
        for field in fields(self):
            t = getattr(self, field.name)
            if t.device != self.q.device or t.dtype not in (torch.float32, torch.bfloat16):
                raise ValueError(f"{field.name} must be FP32/BF16 on the same device as q")
        for name in ("k", "v", "a", "b", "gate"):
            if getattr(self, name).dtype != self.q.dtype:
                raise ValueError(f"{name} must have the same dtype as q")
        if self.a_log.dtype != torch.float32:
            raise ValueError("a_log must be FP32")


@dataclass(frozen=True)
class GDNResult:
    output: Tensor  # [B, T, Hv, V] in the input dtype
    final_state: Tensor  # [B, Hv, V, K] fp32
    checkpoints: Tensor  # [B, T+1, Hv, V, K] (index 0 = initial) or [B, 0, Hv, V, K]


def _unit_rows(x: Tensor) -> Tensor:
    return x * torch.rsqrt(x.square().sum(-1, keepdim=True) + 1e-6)


def post_conv_gdn(
    inputs: GDNInputs,
    initial_state: Tensor,
    lengths: Tensor,
    *,
    save_checkpoints: bool = False,
    norm_eps: float = 1e-6,
) -> GDNResult:
    """Run T tokens of the gated delta rule without mutating any input."""
    inputs.validate()
    if norm_eps <= 0:
        raise ValueError("norm_eps must be positive")
    batch, tokens, key_heads, key_dim = inputs.q.shape
    value_heads, value_dim = inputs.v.shape[-2:]
    if tuple(initial_state.shape) != (batch, value_heads, value_dim, key_dim):
        raise ValueError("initial_state must be [B, Hv, V, K]")
    if initial_state.dtype != torch.float32 or initial_state.device != inputs.q.device:
        raise ValueError("initial_state must be FP32 on the input device")
    if tuple(lengths.shape) != (batch,) or lengths.dtype not in (torch.int32, torch.int64):
        raise ValueError("lengths must be an int32/int64 vector of size B")
    if lengths.device != inputs.q.device:
        raise ValueError("lengths must be on the input device")

    group = value_heads // key_heads
    q_hat = _unit_rows(inputs.q.float()).repeat_interleave(group, dim=2) * key_dim**-0.5
    k_hat = _unit_rows(inputs.k.float()).repeat_interleave(group, dim=2)
    decay = torch.exp(-torch.exp(inputs.a_log) * F.softplus(inputs.a.float() + inputs.dt_bias.float()))
    beta = torch.sigmoid(inputs.b.float())
    v = inputs.v.float()
    weight = inputs.norm_weight.float()
    out_dtype = inputs.q.dtype

    state = initial_state
    saved = [initial_state] if save_checkpoints else []
    outputs = []
    for t in range(tokens):
        live = (lengths > t).view(batch, 1, 1, 1)
        kt = k_hat[:, t, :, None, :]  # [B, Hv, 1, K]
        decayed = state * decay[:, t, :, None, None]
        residual = v[:, t] - (decayed * kt).sum(-1)
        candidate = decayed + (residual * beta[:, t, :, None])[..., None] * kt
        state = torch.where(live, candidate, state)
        raw = (state * q_hat[:, t, :, None, :]).sum(-1).to(out_dtype).float()
        scaled = raw * torch.rsqrt(raw.square().mean(-1, keepdim=True) + norm_eps)
        y = scaled * weight * F.silu(inputs.gate[:, t].float())
        outputs.append(torch.where(live.view(batch, 1, 1), y, 0).to(out_dtype))
        if save_checkpoints:
            saved.append(state)
    checkpoints = (
        torch.stack(saved, dim=1)
        if save_checkpoints
        else initial_state.new_empty((batch, 0, value_heads, value_dim, key_dim))
    )
    return GDNResult(torch.stack(outputs, dim=1), state, checkpoints)
