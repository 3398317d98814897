"""Seeded synthetic decode workloads (inputs only; no computation).

`decode_case` builds the arguments of one `GDNBackend` / `torch.ops.lightdelta.decode` call
with the strided activation layouts the production caller hands over (reference
tests/conftest.py:14-31): qkv and gate are column slices of one [tokens, qkv + gate] buffer,
a and b are column slices of one [tokens, 2*HV] buffer.

Distributions ("workload", seed 0 by default): q, k, v, gate bf16 ~ N(0,1); a, b bf16 ~
N(0,1) (beta = sigmoid(b), log-decay = -softplus(a + dt_bias) * exp(A_log)); A_log fp32 ~
U(-1,1); dt_bias fp32 zeros; norm weight fp32 1 + 0.1 N(0,1); state fp32 0.02 N(0,1).
Request r owns slots[r, :] (distinct random ids in [1, pool_slots); slot 0 is reserved) and
tokens r*width .. r*width + width - 1.
"""

from __future__ import annotations

import torch

HEAD_DIM = 128


def decode_case(
    batch: int,
    width: int = 1,
    *,
    num_k_heads: int = 16,
    num_v_heads: int = 32,
    pool_slots: int | None = None,
    seed: int = 0,
    device="cuda",
    dt_bias_dtype=torch.float32,
    weight_dtype=torch.float32,
    state_std: float = 0.02,
) -> dict:
    gen = torch.Generator(device="cpu").manual_seed(seed)
    n = batch * width
    qkv_cols = (2 * num_k_heads + num_v_heads) * HEAD_DIM
    gate_cols = num_v_heads * HEAD_DIM
    if pool_slots is None:
        pool_slots = n + 1

    def normal(*shape):
        return torch.randn(*shape, generator=gen)

    qkvz = normal(n, qkv_cols + gate_cols).to(torch.bfloat16)
    ba = normal(n, 2 * num_v_heads).to(torch.bfloat16)
    if pool_slots - 1 >= n:
        ids = torch.randperm(pool_slots - 1, generator=gen)[:n] + 1
    else:  # a pool smaller than the batch: slot ids repeat (for callers that replace them)
        ids = torch.randint(1, pool_slots, (n,), generator=gen)
    case = dict(
        qkv=qkvz[:, :qkv_cols],
        a=ba[:, num_v_heads:],
        b=ba[:, :num_v_heads],
        a_log=torch.rand(num_v_heads, generator=gen) * 2 - 1,
        dt_bias=torch.zeros(num_v_heads).to(dt_bias_dtype),
        slots=ids.to(torch.int32).view(batch, width),
        cu=torch.arange(0, n + 1, width, dtype=torch.int32),
        accepted=torch.ones(batch, dtype=torch.int32),
        pool=state_std * normal(pool_slots, num_v_heads, HEAD_DIM, HEAD_DIM),
        gate=qkvz[:, qkv_cols:].view(n, num_v_heads, HEAD_DIM),
        weight=(1 + 0.1 * normal(HEAD_DIM)).to(weight_dtype),
        out=torch.zeros(n, num_v_heads, HEAD_DIM, dtype=torch.bfloat16),
    )
    if torch.device(device).type != "cpu":
        # Move the shared buffers once so the strided views stay views on the device.
        qkvz_d = qkvz.to(device)
        ba_d = ba.to(device)
        moved = {k: v.to(device) for k, v in case.items() if k not in ("qkv", "a", "b", "gate")}
        moved.update(
            qkv=qkvz_d[:, :qkv_cols],
            a=ba_d[:, num_v_heads:],
            b=ba_d[:, :num_v_heads],
            gate=qkvz_d[:, qkv_cols:].view(n, num_v_heads, HEAD_DIM),
        )
        case = moved
    return case


def stack_case(layers: int, batch: int, *, num_k_heads: int = 16, num_v_heads: int = 32,
               pool_slots: int = 1024, seed: int = 0, device="cuda", conv_len: int = 0) -> dict:
    """A stack of `layers` GDN decode layers, one token per request: per-layer activations,
    parameters and state pool (one [layers, pool_slots, HV, 128, 128] fp32 tensor), and one
    slots/cu/accepted set shared by every layer (a request keeps its slot id in every
    layer).  Same distributions as decode_case; generated on `device`.

    conv_len > 0 adds each layer's causal-conv parameters for the conv-fused step (the
    activations are then its pre-conv input): conv_state [layers, pool_slots, conv_dim,
    conv_len] bf16 ~ N(0, 1), dim-first as vLLM allocates it, and conv_weight [layers,
    conv_dim, 4] bf16 ~ N(0, 1/4); no bias.  A request's conv slot is its SSM slot."""
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(seed)
    qkv_cols = (2 * num_k_heads + num_v_heads) * HEAD_DIM
    gate_cols = num_v_heads * HEAD_DIM
    qkvz = torch.randn(layers, batch, qkv_cols + gate_cols, generator=gen, device=dev).bfloat16()
    ba = torch.randn(layers, batch, 2 * num_v_heads, generator=gen, device=dev).bfloat16()
    pool = torch.empty(layers, pool_slots, num_v_heads, HEAD_DIM, HEAD_DIM, device=dev)
    for layer in range(layers):
        pool[layer].normal_(0.0, 0.02, generator=gen)
    cpu_gen = torch.Generator().manual_seed(seed)
    slots = (torch.randperm(pool_slots - 1, generator=cpu_gen)[:batch] + 1).to(torch.int32)
    case = dict(
        qkv=qkvz[:, :, :qkv_cols],
        a=ba[:, :, num_v_heads:],
        b=ba[:, :, :num_v_heads],
        a_log=(torch.rand(layers, num_v_heads, generator=gen, device=dev) * 2 - 1),
        dt_bias=torch.zeros(layers, num_v_heads, device=dev),
        slots=slots.view(batch, 1).to(dev),
        cu=torch.arange(0, batch + 1, dtype=torch.int32, device=dev),
        accepted=torch.ones(batch, dtype=torch.int32, device=dev),
        pool=pool,
        gate=qkvz[:, :, qkv_cols:].unflatten(-1, (num_v_heads, HEAD_DIM)),
        weight=1 + 0.1 * torch.randn(layers, HEAD_DIM, generator=gen, device=dev),
        out=torch.zeros(layers, batch, num_v_heads, HEAD_DIM, dtype=torch.bfloat16, device=dev),
    )
    if conv_len > 0:
        conv_state = torch.empty(layers, pool_slots, qkv_cols, conv_len, dtype=torch.bfloat16,
                                 device=dev)
        for layer in range(layers):  # one layer at a time: the fp32 draw is 4 x the pool
            conv_state[layer] = torch.randn(pool_slots, qkv_cols, conv_len, generator=gen,
                                            device=dev).bfloat16()
        case["conv_state"] = conv_state
        case["conv_weight"] = (torch.randn(layers, qkv_cols, 4, generator=gen, device=dev)
                               / 2).bfloat16()
    return case


STACK_SHARED = ("slots", "cu", "accepted")


def stack_layer(case: dict, layer: int) -> dict:
    """Arguments of layer `layer` of a stack_case, keyed like decode_case."""
    return {k: (v if k in STACK_SHARED else v[layer]) for k, v in case.items()}
