"""A 48-layer stack of decode steps captured as one HIP graph at full size: batch 128,
16 qk / 32 v heads, 1024 slots per layer (96 GiB of fp32 state), slot ids reshuffled
between replays; once with the post-conv decode and once with the conv-fused step (each
layer with its own bf16 conv pool of 1024 slots).  Checked against the oracle on sampled
layers and requests (requests are independent, so a sub-batch of the oracle is exact for
them), and through a per-slot checksum of every slot of every layer (SSM and conv pools):
exactly the slots of the current batch change, in every layer, on every replay."""

from __future__ import annotations

import pytest
import torch

from lightdelta_amd import ops
from lightdelta_amd.workloads import stack_case, stack_layer
from oracle.decode import expected_decode, expected_decode_conv
from tests.parity import assert_bf16_outputs, assert_states

pytestmark = pytest.mark.gpu

LAYERS, BATCH, SLOTS = 48, 128, 1024
ORDER = ("qkv", "a", "b", "a_log", "dt_bias", "slots", "cu", "accepted", "pool", "gate", "weight",
         "out")
CHECKED_LAYERS = (0, 23, 47)
CHECKED_REQUESTS = torch.tensor([0, 37, 64, 127])
# The reference's one-step state tolerance (tests/test_gdn.py:74).
STEP_STATE = dict(rtol=3e-4, atol=3e-6)


def slot_checksums(pool: torch.Tensor) -> torch.Tensor:
    """[layers, slots] int64: the sum of every slot's fp32 bit patterns as integers."""
    layers, slots = pool.shape[:2]
    sums = torch.empty(layers, slots, dtype=torch.int64, device=pool.device)
    step = 64
    for layer in range(layers):
        for s in range(0, slots, step):
            bits = pool[layer, s:s + step].reshape(min(step, slots - s), -1).view(torch.int32)
            sums[layer, s:s + step] = bits.to(torch.int64).sum(1)
    return sums.cpu()


def oracle_sub_batch(layer_args: dict, pre_states: torch.Tensor, eps: float,
                     pre_conv: torch.Tensor | None = None):
    """Expected outputs and states of CHECKED_REQUESTS, from their pre-step states (and, for
    the conv-fused step, their pre-step conv states): (out, pool, pre[, conv_state, post])
    over a mini pool whose slot r + 1 holds checked request r."""
    n = len(CHECKED_REQUESTS)
    rows = CHECKED_REQUESTS
    mini_pool = torch.zeros(n + 1, *pre_states.shape[1:])
    mini_pool[1:] = pre_states
    rest = (layer_args["a"].cpu()[rows], layer_args["b"].cpu()[rows], layer_args["a_log"],
            layer_args["dt_bias"], torch.arange(1, n + 1, dtype=torch.int32).view(n, 1),
            torch.arange(n + 1, dtype=torch.int32), torch.ones(n, dtype=torch.int32), mini_pool,
            layer_args["gate"].cpu()[rows], layer_args["weight"],
            torch.zeros(n, *layer_args["out"].shape[1:], dtype=torch.bfloat16), eps)
    if pre_conv is None:
        return expected_decode(layer_args["qkv"].cpu()[rows], *rest, return_pre=True)
    mini_conv = torch.zeros(n + 1, *pre_conv.shape[1:], dtype=pre_conv.dtype)
    mini_conv[1:] = pre_conv
    return expected_decode_conv(layer_args["qkv"].cpu()[rows], mini_conv,
                                layer_args["conv_weight"].cpu(), None, *rest, return_pre=True)


def run_stack(gpu, conv: bool):
    print(f"case: stack layers={LAYERS} batch={BATCH} slots={SLOTS} conv={conv}", flush=True)
    case = stack_case(LAYERS, BATCH, pool_slots=SLOTS, seed=3 + conv, device=gpu,
                      conv_len=3 if conv else 0)
    layers = [stack_layer(case, layer) for layer in range(LAYERS)]
    eps = 1e-6

    def step():
        for args in layers:
            if conv:
                torch.ops.lightdelta.decode_conv(args["qkv"], args["conv_state"],
                                                 args["conv_weight"], None,
                                                 *[args[k] for k in ORDER[1:]], eps)
            else:
                torch.ops.lightdelta.decode(*[args[k] for k in ORDER], eps)

    policy = ops.state_cache_policy()
    ops.set_state_cache_policy("stream")  # 96 GiB of state: nothing stays cached
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()  # eager warm-up (also a first step of the stack)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
    finally:
        ops.set_state_cache_policy(policy)
    torch.cuda.synchronize()

    pools = {"SSM": case["pool"]}
    if conv:
        pools["conv"] = case["conv_state"]
    gen = torch.Generator().manual_seed(4)
    for replay in range(3):
        ids = (torch.randperm(SLOTS - 1, generator=gen)[:BATCH] + 1).to(torch.int32)
        case["slots"].copy_(ids.view(BATCH, 1))
        checked_slots = ids[CHECKED_REQUESTS].long()
        at = checked_slots.to(gpu)
        pre = {layer: case["pool"][layer, at].cpu() for layer in CHECKED_LAYERS}
        pre_conv = {layer: (case["conv_state"][layer, at].cpu() if conv else None)
                    for layer in CHECKED_LAYERS}
        before = {name: slot_checksums(pool) for name, pool in pools.items()}
        graph.replay()
        torch.cuda.synchronize()

        active = torch.zeros(SLOTS, dtype=torch.bool)
        active[ids.long()] = True
        for name, pool in pools.items():
            changed = before[name] != slot_checksums(pool)
            assert not changed[:, ~active].any(), \
                f"replay {replay}: a {name} slot outside the batch changed"
            assert changed[:, active].all(), f"replay {replay}: a batch {name} slot was not written"

        for layer in CHECKED_LAYERS:
            expected = oracle_sub_batch(layers[layer], pre[layer], eps, pre_conv[layer])
            exp_out, exp_states, pre_vals = expected[:3]
            label = f"replay {replay} layer {layer}"
            got_out = case["out"][layer, CHECKED_REQUESTS.to(gpu)].cpu()
            assert_bf16_outputs(got_out, exp_out, pre_vals, label=label)
            got_states = case["pool"][layer, at].cpu()
            assert_states(got_states, exp_states[1:], label=label, **STEP_STATE)
            if conv:
                got_conv = case["conv_state"][layer, at].cpu()
                assert torch.equal(got_conv, expected[3][1:]), f"{label}: conv state differs"


def test_48_layer_graph_with_reshuffled_slots(gpu):
    run_stack(gpu, conv=False)


def test_48_layer_conv_fused_graph_with_reshuffled_slots(gpu):
    """The serving layer's step: one decode_conv launch per layer, each layer with its own
    1024-slot conv pool; the conv states of the checked requests are bit-exact."""
    run_stack(gpu, conv=True)
