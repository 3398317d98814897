"""Parity of the conv-fused decode (torch.ops.lightdelta.decode_conv) with the oracle's
composition: conv update (oracle/conv.py) then the GDN step (oracle/decode.py).  The conv
state is a pure shift of bf16 data and must match bit for bit; SSM states and outputs follow
the decode tolerances.  Covers the workload's first configuration (B=1, 4/8 heads,
zero-initialised conv state), the k-head groups 1, 2 and 3 (direct write and the
last-reader write of the shared q/k conv state), vLLM's dim-first and dim-last conv pools,
the kernel's packed conv-state path against its per-element path, state lengths 3, 4 and 6,
bias, padding and zero-token requests, speculative verify with 2 to 4 tokens and random
accepted counts over consecutive steps, requests the conv rejects, and graph replay.  The
single-token cases run under both state cache policies, which launch different shapes."""

from __future__ import annotations

import pytest
import torch

from lightdelta_amd import ops
from lightdelta_amd.workloads import decode_case
from oracle.decode import expected_decode_conv
from tests.parity import assert_bf16_outputs, assert_states

pytestmark = pytest.mark.gpu

ORDER = ("a", "b", "a_log", "dt_bias", "slots", "cu", "accepted", "pool", "gate", "weight", "out")
# The reference's one-step state tolerance (tests/test_gdn.py:74).
STEP_STATE = dict(rtol=3e-4, atol=3e-6)


def announce(**what):
    print("case:", " ".join(f"{k}={v}" for k, v in what.items()), flush=True)


@pytest.fixture(params=["keep", "stream"])
def policy(request):
    """Runs the test under each state cache policy: a single-token step launches 4 waves per
    workgroup (its conv state moved as packed pieces when aligned) under keep and 16 waves
    (one conv channel per thread) under stream."""
    saved = ops.state_cache_policy()
    ops.set_state_cache_policy(request.param)
    yield request.param
    ops.set_state_cache_policy(saved)


def conv_case(gpu, batch, heads, pool_slots, length=3, dim_last=False, bias=False, seed=0,
              zero_state=False, width=1):
    case = decode_case(batch, width, num_k_heads=heads[0], num_v_heads=heads[1],
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
    got_conv = case["conv_state"].cpu()
    if not torch.equal(got_conv, exp_conv):
        bad = (got_conv != exp_conv).nonzero()
        raise AssertionError(f"{label}: conv state differs at {len(bad)} elements "
                             f"(slot, channel, column) first {bad[:6].tolist()}")
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


@pytest.mark.parametrize("heads", [(16, 16), (16, 32), (16, 48), (8, 16)])
def test_head_groups_and_shared_conv_state(gpu, heads, policy):
    announce(test="conv_groups", heads=heads, policy=policy)
    case = conv_case(gpu, 8, heads, pool_slots=12, seed=heads[1])
    run_and_check(case, 3, torch.Generator().manual_seed(2), label=f"heads {heads}")


@pytest.mark.parametrize("dim_last,length,bias", [(False, 4, True), (True, 3, False), (True, 4, True)])
def test_conv_pool_layouts(gpu, dim_last, length, bias, policy):
    announce(test="conv_layouts", dim_last=dim_last, length=length, bias=bias, policy=policy)
    case = conv_case(gpu, 6, (16, 32), pool_slots=10, length=length, dim_last=dim_last,
                     bias=bias, seed=length)
    run_and_check(case, 3, torch.Generator().manual_seed(3), label="layout")


def test_workload_batch(gpu):
    """B=32, 16 qk / 32 v heads, 256-slot pools."""
    announce(test="conv_b32")
    case = conv_case(gpu, 32, (16, 32), pool_slots=256, seed=5)
    run_and_check(case, 4, torch.Generator().manual_seed(4), label="b32")


def test_padding_and_empty_requests(gpu, policy):
    announce(test="conv_padding", policy=policy)
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


@pytest.mark.parametrize("width,heads,dim_last", [(2, (16, 32), False), (3, (16, 16), True),
                                                  (4, (16, 32), True), (4, (16, 48), False)])
def test_speculative_verify_steps(gpu, width, heads, dim_last):
    """Consecutive verify steps with W tokens per request and a conv state of 3 + W - 1
    columns; each step's accepted count (the previous step's accepted tokens) is random in
    1..W, so the conv history starts at a different column per request."""
    announce(test="conv_verify", width=width, heads=heads, dim_last=dim_last)
    case = conv_case(gpu, 6, heads, pool_slots=6 * width + 2, length=3 + width - 1,
                     dim_last=dim_last, bias=True, seed=20 + width, width=width)
    gen = torch.Generator().manual_seed(30 + width)
    for step in range(3):
        case["accepted"].copy_(torch.randint(1, width + 1, (6,), generator=gen, dtype=torch.int32))
        run_and_check(case, 1, gen, label=f"verify W={width} step {step}")


def test_ragged_verify_and_rejected_requests(gpu):
    """W=4 with requests of 4, 2, 1 and 3 tokens: accepted within each request's tokens, one
    request whose accepted count exceeds its tokens (its kept conv columns would fall
    outside the state: rejected, zero outputs), one whose conv slot indices[r, 0] is padding
    while its source slot is valid (rejected), and a padding-free short request."""
    announce(test="conv_ragged")
    case = conv_case(gpu, 6, (16, 32), pool_slots=30, length=6, seed=40, width=4)
    case["cu"].copy_(torch.tensor([0, 4, 6, 7, 10, 12, 14], device=gpu, dtype=torch.int32))
    case["accepted"].copy_(torch.tensor([3, 2, 1, 3, 2, 2], device=gpu, dtype=torch.int32))
    case["accepted"][3] = 3  # 3 tokens, accepted 3: valid
    case["accepted"][4] = 2  # 2 tokens, accepted 2: valid
    case["cu"][5] = 13
    case["accepted"][5] = 2  # request 5 has 1 token (13..14) and accepted 2 > 1: rejected
    case["slots"][1, 0] = 0  # request 1: conv slot padding, source slots[1, 1] valid: rejected
    for name in ("qkv", "a", "b", "gate", "out"):
        case[name] = case[name][:14]
    case["out"].fill_(1.0)
    before = case["conv_state"].clone()
    run_and_check(case, 1, torch.Generator().manual_seed(41), label="ragged verify")
    out = case["out"].float().cpu()
    assert out[4:6].abs().sum() == 0 and out[13:14].abs().sum() == 0
    for r in (1, 5):
        s0 = int(case["slots"][r, 0])
        if s0 > 0:
            assert torch.equal(case["conv_state"][s0].cpu(), before[s0].cpu())


@pytest.mark.parametrize("length,heads,bias", [(3, (16, 32), False), (4, (4, 8), True),
                                                 (3, (16, 48), True)])
def test_packed_and_per_element_conv_paths_agree(gpu, length, heads, bias, policy):
    """A dense, 16-byte aligned dim-first conv pool takes the kernel's packed path (each wave
    moves its channels' columns as 16-byte pieces: 4 waves with a q/k and a v run each under
    the keep policy, waves 0..5 of 16 with one run each under the stream policy); the same
    data one element into a larger buffer (2-byte aligned) takes the per-element path, which
    loads each column as one element and needs no alignment beyond the element's.  Over 3
    steps both give the same bits for the conv state, the SSM pool and the outputs, and the
    aligned run matches the oracle."""
    announce(test="conv_packed_vs_per_element", length=length, heads=heads, bias=bias,
             policy=policy)
    case = conv_case(gpu, 8, heads, pool_slots=10, length=length, bias=bias, seed=90 + length)
    dense = case["conv_state"]
    flat = torch.empty(dense.numel() + 1, dtype=dense.dtype, device=dense.device)
    shifted = flat[1:].view(dense.shape)
    shifted.copy_(dense)
    assert dense.data_ptr() % 16 == 0 and shifted.data_ptr() % 16 != 0
    pool2, out2 = case["pool"].clone(), case["out"].clone()
    gen = torch.Generator().manual_seed(93)
    for step in range(3):
        case["qkv"].copy_(torch.randn(case["qkv"].shape, generator=gen).bfloat16())
        expected = expected_decode_conv(
            case["qkv"], dense, case["conv_weight"], case["conv_bias"],
            *[case[k] for k in ORDER], 1e-6, return_pre=True)
        rest = [case[k] for k in ORDER]
        torch.ops.lightdelta.decode_conv(case["qkv"], dense, case["conv_weight"],
                                         case["conv_bias"], *rest, 1e-6)
        rest[ORDER.index("pool")], rest[ORDER.index("out")] = pool2, out2
        torch.ops.lightdelta.decode_conv(case["qkv"], shifted, case["conv_weight"],
                                         case["conv_bias"], *rest, 1e-6)
        torch.cuda.synchronize()
        assert torch.equal(dense, shifted), f"step {step}: conv states differ between the paths"
        assert torch.equal(case["pool"], pool2), f"step {step}: SSM pools differ between the paths"
        assert torch.equal(case["out"], out2), f"step {step}: outputs differ between the paths"
        check_step(case, expected, f"packed step {step}")
        case["pool"].copy_(expected[1].to(case["pool"].device))
        pool2.copy_(case["pool"])


def test_single_token_long_conv_state(gpu, policy):
    """One token per request with a 6-column conv state (the conv runs before the tile)."""
    announce(test="conv_long_state", policy=policy)
    case = conv_case(gpu, 8, (16, 32), pool_slots=12, length=6, bias=True, seed=50)
    run_and_check(case, 3, torch.Generator().manual_seed(51), label="long state")


def test_verify_graph_replay(gpu):
    announce(test="conv_verify_graph")
    case = conv_case(gpu, 4, (16, 32), pool_slots=20, length=6, seed=60, width=4)
    case["accepted"].copy_(torch.tensor([1, 4, 2, 3], device=gpu, dtype=torch.int32))
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
    gen = torch.Generator().manual_seed(61)
    for replay in range(3):
        case["qkv"].copy_(torch.randn(case["qkv"].shape, generator=gen).bfloat16())
        case["accepted"].copy_(torch.randint(1, 5, (4,), generator=gen, dtype=torch.int32))
        expected = expected_decode_conv(*args(), return_pre=True)
        graph.replay()
        torch.cuda.synchronize()
        check_step(case, expected, f"verify replay {replay}")
        case["pool"].copy_(expected[1].to(case["pool"].device))


@pytest.mark.parametrize("batch,width,steps", [(32, 1, 64), (8, 3, 16)])
def test_drift_without_resync(gpu, batch, width, steps, policy):
    """The GPU carries its own SSM and conv pools for `steps` consecutive steps (no copy of
    the oracle's state back into the GPU pool), the oracle its own trajectory from the same
    inputs: the conv state stays bit-exact, every step's outputs meet the decode tolerance
    and the SSM pool stays within rtol = atol = 2e-3 of the oracle's at the end.  With
    width > 1, every step's accepted count is random in 1..width, so the source state and
    the conv history come from different per-token slots and columns each step."""
    announce(test="conv_drift", batch=batch, width=width, steps=steps, policy=policy)
    case = conv_case(gpu, batch, (16, 32), pool_slots=batch * width + 2, length=3 + width - 1,
                     bias=width > 1, seed=70 + width, width=width)
    cpu = {k: (None if v is None else v.cpu().clone()) for k, v in case.items()}
    gen = torch.Generator().manual_seed(71 + width)
    flips = 0
    for step in range(steps):
        fresh = torch.randn(case["qkv"].shape, generator=gen).bfloat16()
        case["qkv"].copy_(fresh.to(gpu))
        cpu["qkv"] = fresh
        if width > 1:
            acc = torch.randint(1, width + 1, (batch,), generator=gen, dtype=torch.int32)
            case["accepted"].copy_(acc.to(gpu))
            cpu["accepted"] = acc
        exp_out, exp_pool, pre, exp_conv, _ = expected_decode_conv(
            cpu["qkv"], cpu["conv_state"], cpu["conv_weight"], cpu["conv_bias"],
            *[cpu[k] for k in ORDER], 1e-6, return_pre=True)
        torch.ops.lightdelta.decode_conv(case["qkv"], case["conv_state"], case["conv_weight"],
                                         case["conv_bias"], *[case[k] for k in ORDER], 1e-6)
        torch.cuda.synchronize()
        if not torch.equal(case["conv_state"].cpu(), exp_conv):
            raise AssertionError(f"drift step {step}: conv state differs")
        flips += assert_bf16_outputs(case["out"], exp_out, pre, label=f"drift step {step}")["flips"]
        cpu["pool"], cpu["conv_state"], cpu["out"] = exp_pool, exp_conv, exp_out
    assert_states(case["pool"], cpu["pool"], label=f"SSM pool after {steps} steps")
    print(f"conv drift B={batch} W={width}: {flips} rounding flips over {steps} steps")
