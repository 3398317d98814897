"""Parity of the conv-fused decode (torch.ops.lightdelta.decode_conv) with the oracle's
composition: conv update (oracle/conv.py) then the GDN step (oracle/decode.py).  The conv
state is a pure shift of bf16 data and must match bit for bit; SSM states and outputs follow
the decode tolerances.  Covers the workload's first configuration (B=1, 4/8 heads,
zero-initialised conv state), the k-head groups 1, 2 and 3 (direct write and the
last-reader write of the shared q/k conv state), vLLM's dim-first and dim-last conv pools,
state lengths 3 and 4, bias, padding and zero-token requests, and graph replay."""

from __future__ import annotations

import pytest
import torch

from lightdelta_amd.workloads import decode_case
from oracle.decode import expected_decode_conv
from tests.parity import assert_bf16_outputs, assert_states

pytestmark = pytest.mark.gpu

ORDER = ("a", "b", "a_log", "dt_bias", "slots", "cu", "accepted", "pool", "gate", "weight", "out")
# The reference's one-step state tolerance (tests/test_gdn.py:74).
STEP_STATE = dict(rtol=3e-4, atol=3e-6)


def announce(**what):
    print("case:", " ".join(f"{k}={v}" for k, v in what.items()), flush=True)


def conv_case(gpu, batch, heads, pool_slots, length=3, dim_last=False, bias=False, seed=0,
              zero_state=False):
    case = decode_case(batch, 1, num_k_heads=heads[0], num_v_heads=heads[1],
                       pool_slots=pool_slots, seed=seed, device=gpu)
    conv_dim = case["qkv"].shape[1]
    g = torch.Generator().manual_seed(seed + 100)
    if dim_last:
        storage = torch.randn(pool_slots, length, conv_dim, generator=g).bfloat16()
        conv_state = storage.to(gpu).transpose(1, 2)  # [slots, conv_dim, length] view
    else:
        conv_state = torch.randn(pool_slots, conv_dim, length, generator=g).bfloat16().to(gpu)
    if zero_state:
        conv_state.zero_()
    case["conv_state"] = conv_state
    case["conv_weight"] = (torch.randn(conv_dim, 4, generator=g) / 2).bfloat16().to(gpu)
    case["conv_bias"] = (torch.randn(conv_dim, generator=g).bfloat16().to(gpu) if bias else None)
    return case


def check_step(case, expected, label):
    """The conv output is correctly rounded on both sides, so the post-conv activations are
    bit-identical and the GDN step is held to the plain decode tolerances."""
    exp_out, exp_pool, pre, exp_conv, _ = expected
    assert torch.equal(case["conv_state"].cpu(), exp_conv), f"{label}: conv state"
    assert_bf16_outputs(case["out"], exp_out, pre, label=label)
    assert_states(case["pool"], exp_pool, label=label, **STEP_STATE)


def run_and_check(case, steps, gen, eps=1e-6, label=""):
    for step in range(steps):
        case["qkv"].copy_(torch.randn(case["qkv"].shape, generator=gen).bfloat16())
        expected = expected_decode_conv(
            case["qkv"], case["conv_state"], case["conv_weight"], case["conv_bias"],
            *[case[k] for k in ORDER], eps, return_pre=True)
        torch.ops.lightdelta.decode_conv(case["qkv"], case["conv_state"], case["conv_weight"],
                                         case["conv_bias"], *[case[k] for k in ORDER], eps)
        torch.cuda.synchronize()
        check_step(case, expected, f"{label} step {step}")
        # continue from the oracle's trajectory so every step is checked from equal inputs
        case["pool"].copy_(expected[1].to(case["pool"].device))


def test_first_workload_config_zero_conv_state(gpu):
    """B=1, 4 qk / 8 v heads, zero-initialised conv state, 16 consecutive steps."""
    announce(test="conv_cfg1")
    case = conv_case(gpu, 1, (4, 8), pool_slots=3, zero_state=True)
    run_and_check(case, 16, torch.Generator().manual_seed(1), label="cfg1")


@pytest.mark.parametrize("heads", [(16, 16), (16, 32), (16, 48)])
def test_head_groups_and_shared_conv_state(gpu, heads):
    announce(test="conv_groups", heads=heads)
    case = conv_case(gpu, 8, heads, pool_slots=12, seed=heads[1])
    run_and_check(case, 3, torch.Generator().manual_seed(2), label=f"heads {heads}")


@pytest.mark.parametrize("dim_last,length,bias", [(False, 4, True), (True, 3, False), (True, 4, True)])
def test_conv_pool_layouts(gpu, dim_last, length, bias):
    announce(test="conv_layouts", dim_last=dim_last, length=length, bias=bias)
    case = conv_case(gpu, 6, (16, 32), pool_slots=10, length=length, dim_last=dim_last,
                     bias=bias, seed=length)
    run_and_check(case, 3, torch.Generator().manual_seed(3), label="layout")


def test_workload_batch(gpu):
    """B=32, 16 qk / 32 v heads, 256-slot pools."""
    announce(test="conv_b32")
    case = conv_case(gpu, 32, (16, 32), pool_slots=256, seed=5)
    run_and_check(case, 4, torch.Generator().manual_seed(4), label="b32")


def test_padding_and_empty_requests(gpu):
    announce(test="conv_padding")
    case = conv_case(gpu, 4, (16, 32), pool_slots=8, seed=6)
    case["slots"][1, 0] = 0  # padding request
    case["cu"].copy_(torch.tensor([0, 1, 2, 2, 3], device=gpu, dtype=torch.int32))  # request 2 empty
    for name in ("qkv", "a", "b", "gate", "out"):
        case[name] = case[name][:3]
    before = case["conv_state"].clone()
    run_and_check(case, 2, torch.Generator().manual_seed(5), label="padding")
    padded = int(case["slots"][1, 0])
    assert torch.equal(case["conv_state"][padded].cpu(), before[padded].cpu())


def test_graph_replay_with_changed_slots(gpu):
    announce(test="conv_graph")
    case = conv_case(gpu, 4, (16, 32), pool_slots=12, seed=7)
    args = lambda: (case["qkv"], case["conv_state"], case["conv_weight"], case["conv_bias"],  # noqa: E731
                    *[case[k] for k in ORDER], 1e-6)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        torch.ops.lightdelta.decode_conv(*args())
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        torch.ops.lightdelta.decode_conv(*args())
    free = [s for s in range(1, 12) if s not in case["slots"].flatten().tolist()]
    case["slots"].copy_(torch.tensor(free[:4], device=gpu, dtype=torch.int32).view(4, 1))
    gen = torch.Generator().manual_seed(8)
    for replay in range(3):
        case["qkv"].copy_(torch.randn(case["qkv"].shape, generator=gen).bfloat16())
        expected = expected_decode_conv(*args(), return_pre=True)
        graph.replay()
        torch.cuda.synchronize()
        check_step(case, expected, f"replay {replay}")
        case["pool"].copy_(expected[1].to(case["pool"].device))
