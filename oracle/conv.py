"""Causal depthwise conv1d update of decode tokens -- test infrastructure.

The pre-GDN step of the decode layer: vLLM 0.29 `causal_conv1d_update`, called at the
reference's python/lightdelta/integration/vllm_layer.py:199-207 (one token per request)
and :161-172 (MTP verify: `num_accepted_tokens`, `query_start_loc`).  vLLM is a third-party
dependency absent here, so this restates its published algorithm.  Per request with L new
tokens x_0 .. x_{L-1}, conv state of S columns and offset a = num_accepted_tokens - 1
(0 without speculative decoding), per channel d:

  history   h = state[d, a .. a+W-2]                    (the W-1 inputs before x_0)
  sequence  q = h ++ [x_0, .., x_{L-1}]
  acc_t     = bias[d]; acc_t = fma(weight[d, j], q[t + j], acc_t) for j = 0 .. W-1
  y_t[d]    = bf16( silu(acc_t) )                       (fp32 accumulation, oldest tap first)
  new state = [state[d, a+1 .. a+S-L], x_0, .., x_{L-1}] (S columns: the state after the
                                                         first token of the step, then the
                                                         step's inputs)

With L = 1 and a = 0 this is the plain shift: state[d, 1 .. S-1] then x_0, with the history
in columns 0 .. W-2 whatever S is (vLLM's non-speculative update; S = W-1 there).  The next
step's offset selects, among the S columns, the W-1 inputs that end at its last accepted
token.

The fp32 fused multiply-add chain is emulated exactly in float64 (a product of two fp32
values is exact in float64 and the single rounding back to fp32 is that of an fma).  The
SiLU is evaluated in float64 and rounded once, to the nearest bf16 (ties to even): the
exact value's rounding.  Any fp32 SiLU rounds to the same bf16 except within a few fp32
ulps of a bf16 rounding midpoint, where implementations legitimately differ; fixing the
exact rounding makes the conv output a deterministic function of its inputs.

State layout `[D, S]` per slot (dim-first); a dim-last pool is passed transposed.

The conv arithmetic is pinned: it is checked against torch.nn.functional.conv1d with
groups = D, against an element loop and a brute-force single rounding to bf16, planted
mistakes (reversed taps, a shifted window, a dropped bias, a missing SiLU) fail those
checks, and the multi-token form matches repeated single-token updates.  The standard
non-speculative layout (S = W - 1 = 3 columns, one token, offset 0) is also checked against
transformers' Qwen3-Next statement of the update (modeling_qwen3_next.causal_conv1d_update,
an independent implementation): same state bits, outputs its fp32 conv rounded to bf16.
What stays parity unpinned is vLLM's column convention for speculative steps and longer
states (num_accepted_tokens: which columns hold a step's history, the state left after a
multi-token step): it is restated from vLLM's published algorithm, and no reference test,
fixture or vLLM run here checks it.
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
    """The single-token primitive on an explicit window: x [B, D] (bf16); state [B, D, L]
    whose last W-1 columns are the inputs before x; weight [D, W]; bias [D] or None.
    Returns (y [B, D] bf16, new_state [B, D, L]: shifted left by one, x appended).
    conv_update_tokens applies it to the history columns vLLM selects."""
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


def conv_update_tokens(x: torch.Tensor, state: torch.Tensor, weight: torch.Tensor, bias=None,
                       offset: int = 0):
    """One request's step: x [L, D] (bf16) new tokens, state [D, S] its conv state, offset
    = num_accepted_tokens - 1.  Returns (y [L, D] bf16, new_state [D, S]).  Requires
    offset + W - 2 <= S - 1 and, when S > L, offset + S - L <= S - 1."""
    width = weight.shape[1]
    length = x.shape[0]
    cols = state.shape[-1]
    assert offset + width - 2 <= cols - 1
    assert cols <= length or offset + cols - length <= cols - 1
    history = state[:, offset:offset + width - 1]
    seq = torch.cat([history, x.t().to(state.dtype)], -1)  # [D, W-1+L]
    ys = []
    for t in range(length):
        window = seq[:, t:t + width]  # [D, W]: W-1 inputs before token t, then token t
        y, _ = conv_update(window[:, -1][None].to(x.dtype), window[None, :, :-1], weight, bias)
        ys.append(y[0])
    kept = state[:, offset + 1:offset + 1 + max(cols - length, 0)]
    new_state = torch.cat([kept, x.t().to(state.dtype)], -1)[:, -cols:]
    return torch.stack(ys), new_state
