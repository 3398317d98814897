"""Parity of the gfx950 fused decode against the oracle, through torch.ops.lightdelta and
GDNBackend (which call the C ABI).  Mirrors the reference's GPU tests
(tests/test_gdn.py:58-122) and extends them to the workload shapes (16/32 heads, B=32, 64
steps; MTP verify B=64 T=4 with commit)."""

from __future__ import annotations

import pytest
import torch

from lightdelta_amd import ops
from lightdelta_amd.backend import GDNBackend
from lightdelta_amd.config import BackendConfig
from lightdelta_amd.workloads import decode_case
from oracle import state_io as oracle_state_io
from oracle.decode import expected_decode, packed_reference_step
from tests.parity import assert_bf16_outputs, assert_states

pytestmark = pytest.mark.gpu

ORDER = ("qkv", "a", "b", "a_log", "dt_bias", "slots", "cu", "accepted", "pool", "gate",
         "weight", "out")
# The reference's one-step state tolerance (tests/test_gdn.py:74).
STEP_STATE = dict(rtol=3e-4, atol=3e-6)


def args_of(case):
    return [case[k] for k in ORDER]


def fused(state_io):
    return GDNBackend(BackendConfig(compute="cuda_fused", state_io=state_io))


def expected(case, eps=1e-6):
    return expected_decode(*args_of(case), eps, return_pre=True)


def announce(**what):
    print("case:", " ".join(f"{k}={v}" for k, v in what.items()), flush=True)


@pytest.fixture(params=["keep", "stream"])
def policy(request):
    """Runs the test under each state cache policy (their store paths differ for tokens
    without a destination slot)."""
    saved = ops.state_cache_policy()
    ops.set_state_cache_policy(request.param)
    yield request.param
    ops.set_state_cache_policy(saved)


@pytest.mark.parametrize("heads", [(16, 48), (16, 32), (8, 16), (4, 8), (8, 8)])
@pytest.mark.parametrize("width", [1, 2, 3, 4])
@pytest.mark.parametrize("state_io", ["indexed", "packed"])
def test_matches_oracle(gpu, heads, width, state_io, policy):
    announce(test="matches_oracle", heads=heads, width=width, state_io=state_io, policy=policy)
    case = decode_case(4, width, num_k_heads=heads[0], num_v_heads=heads[1], pool_slots=4 * width + 2,
                       seed=width, device=gpu)
    case["accepted"][:] = torch.arange(4, device=gpu) % width + 1
    case["slots"][-1] = 0  # padding request
    exp_out, exp_pool, pre = expected(case)
    before = case["pool"].clone()
    fused(state_io)(*args_of(case))
    torch.cuda.synchronize()
    assert_bf16_outputs(case["out"], exp_out, pre)
    assert_states(case["pool"], exp_pool, **STEP_STATE)
    assert torch.equal(case["pool"][0], before[0])


@pytest.mark.parametrize("width", [1, 4])
def test_cache_policies_give_identical_bits(gpu, width):
    """The keep and stream policies differ in cache hints and, for one token, in the
    kernel's shape (4 waves of 32 V rows per tile, or 16 of 8): eight consecutive steps at
    the workload shape from the same pool give the same outputs and states bit for bit."""
    announce(test="policies_identical", width=width)
    case = decode_case(32, width, num_k_heads=16, num_v_heads=32, pool_slots=32 * width + 2,
                       seed=40 + width, device=gpu)
    pool0 = case["pool"].clone()
    saved = ops.state_cache_policy()
    results = {}
    try:
        for policy in ("keep", "stream"):
            ops.set_state_cache_policy(policy)
            case["pool"].copy_(pool0)
            outs = []
            for _ in range(8):
                torch.ops.lightdelta.decode(*args_of(case), 1e-6)
                outs.append(case["out"].clone())
            torch.cuda.synchronize()
            results[policy] = (torch.stack(outs), case["pool"].clone())
    finally:
        ops.set_state_cache_policy(saved)
    assert torch.equal(results["keep"][0], results["stream"][0])
    assert torch.equal(results["keep"][1], results["stream"][1])


@pytest.mark.parametrize("dt_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("w_dtype", [torch.float32, torch.bfloat16])
def test_parameter_dtypes(gpu, dt_dtype, w_dtype):
    announce(test="parameter_dtypes", dt=dt_dtype, w=w_dtype)
    case = decode_case(8, 1, pool_slots=20, seed=3, device=gpu, dt_bias_dtype=dt_dtype,
                       weight_dtype=w_dtype)
    case["dt_bias"].copy_(torch.randn(32, device=gpu).to(dt_dtype))
    exp_out, exp_pool, pre = expected(case, eps=1e-5)
    torch.ops.lightdelta.decode(*args_of(case), 1e-5)
    torch.cuda.synchronize()
    assert_bf16_outputs(case["out"], exp_out, pre)
    assert_states(case["pool"], exp_pool, **STEP_STATE)


@pytest.mark.parametrize("state_io", ["packed", "indexed"])
def test_graph_replay_changed_state_indices(gpu, state_io):
    """Capture once, then change slots and accepted in place and replay (reference
    tests/test_gdn.py:78-102)."""
    announce(test="graph_replay", state_io=state_io)
    case = decode_case(2, 3, pool_slots=9, seed=5, device=gpu)
    backend = fused(state_io)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            backend(*args_of(case))
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        backend(*args_of(case))
    case["slots"].copy_(case["slots"].flip(0))
    case["accepted"].fill_(2)
    for replay in range(3):
        before = case["pool"].clone()
        exp_out, exp_pool, pre = expected(case)
        graph.replay()
        torch.cuda.synchronize()
        assert_bf16_outputs(case["out"], exp_out, pre, label=f"replay {replay}")
        assert_states(case["pool"], exp_pool, **STEP_STATE)
        case["pool"].copy_(before)


@pytest.mark.parametrize("state_io", ["packed", "indexed"])
def test_ragged_verification_and_discarded_slots(gpu, state_io, policy):
    """cu=[0,4,7,8,8], an invalid accepted and a discarded candidate slot (reference
    tests/test_gdn.py:105-122)."""
    announce(test="ragged", state_io=state_io, policy=policy)
    case = decode_case(4, 4, pool_slots=18, seed=6, device=gpu)
    case["cu"].copy_(torch.tensor([0, 4, 7, 8, 8], device=gpu, dtype=torch.int32))
    case["accepted"][:] = torch.tensor([0, 3, 1, 2], device=gpu, dtype=torch.int32)
    case["slots"][1, 2] = 0
    for name in ("qkv", "a", "b", "gate", "out"):
        case[name] = case[name][:8]
    case["out"].fill_(1.0)
    exp_out, exp_pool, pre = expected(case)
    fused(state_io)(*args_of(case))
    torch.cuda.synchronize()
    assert_bf16_outputs(case["out"], exp_out, pre)
    assert_states(case["pool"], exp_pool, **STEP_STATE)
    assert case["out"][:4].float().abs().sum() == 0  # invalid accepted -> zero output


def test_invalid_and_empty_requests(gpu, policy):
    """Padding sources (0 and -1), accepted out of range, a zero-token request and an empty
    batch: zero outputs, pool untouched where nothing is valid."""
    announce(test="invalid_and_empty", policy=policy)
    case = decode_case(4, 2, pool_slots=12, seed=7, device=gpu)
    case["slots"][0] = torch.tensor([-1, 0], device=gpu, dtype=torch.int32)
    case["accepted"][:] = torch.tensor([1, 3, 2, 1], device=gpu, dtype=torch.int32)
    case["cu"].copy_(torch.tensor([0, 2, 4, 4, 6], device=gpu, dtype=torch.int32))
    before = case["pool"].clone()
    case["out"].fill_(3.0)
    exp_out, exp_pool, pre = expected(case)
    torch.ops.lightdelta.decode(*args_of(case), 1e-6)
    torch.cuda.synchronize()
    assert_bf16_outputs(case["out"], exp_out, pre)
    assert_states(case["pool"], exp_pool, **STEP_STATE)
    assert torch.equal(case["pool"][0], before[0])
    # empty batch: a no-op
    empty = dict(case)
    empty["slots"] = case["slots"][:0]
    empty["cu"] = case["cu"][:1]
    empty["accepted"] = case["accepted"][:0]
    torch.ops.lightdelta.decode(*args_of(empty), 1e-6)
    torch.cuda.synchronize()


@pytest.mark.parametrize("batch,width", [(1, 1), (7, 2), (33, 3), (100, 4)])
def test_packed_plan_matches_the_reference_bookkeeping(gpu, batch, width):
    """packed_plan (the fused packed path's bookkeeping in one launch) against the reference
    backend's Torch index arithmetic (python/lightdelta/backend.py:39-47, 87-91), on random
    metadata with every edge: accepted 0, -1 and past the width, padding slots 0 and -1
    (also as the source), and requests of 0 .. width tokens."""
    announce(test="packed_plan", batch=batch, width=width)
    gen = torch.Generator().manual_seed(batch * 10 + width)
    slots = torch.randint(-1, 50, (batch, width), generator=gen, dtype=torch.int32)
    accepted = torch.randint(-1, width + 2, (batch,), generator=gen, dtype=torch.int32)
    lengths = torch.randint(0, width + 1, (batch,), generator=gen, dtype=torch.int32)
    cu = torch.zeros(batch + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lengths, 0)
    source = slots.gather(1, (accepted.clamp(1, width) - 1)[:, None].long()).flatten()
    valid = (accepted > 0) & (accepted <= width) & (source > 0)
    live = torch.arange(width)[None, :] < lengths[:, None]
    destinations = torch.where(live & valid[:, None] & (slots > 0), slots, 0).flatten()
    indices = torch.where(valid[:, None], torch.arange(1, 1 + batch * width,
                                                       dtype=torch.int32).view(batch, width), 0)
    out = (torch.full((batch,), -7, dtype=torch.int32, device=gpu),
           torch.ones(batch, dtype=torch.bool, device=gpu),
           torch.full((batch, width), -7, dtype=torch.int32, device=gpu),
           torch.full((batch * width,), -7, dtype=torch.int32, device=gpu))
    torch.ops.lightdelta.packed_plan(slots.to(gpu), cu.to(gpu), accepted.to(gpu), *out)
    torch.cuda.synchronize()
    for name, got, want in zip(("source", "valid", "indices", "destinations"), out,
                               (source, valid, indices, destinations)):
        assert torch.equal(got.cpu(), want.to(got.dtype)), name


def test_workload_64_steps(gpu, policy):
    """Qwen3-Next-shape layer: B=32, 16 qk / 32 v heads, 256-slot pool, random distinct
    slots, 64 consecutive in-place steps.  States and every step's outputs against the
    oracle's own 64-step trajectory (the reference's packed Torch path).  Under each cache
    policy: keep runs the headline kernel (4 waves, plain loads and stores), stream the
    16-wave kernel."""
    announce(test="workload_64_steps", policy=policy)
    case = decode_case(32, 1, pool_slots=256, seed=0, device=gpu)
    cpu = {k: v.cpu().clone() for k, v in case.items()}
    gen = torch.Generator().manual_seed(11)
    flips = 0
    scratch = cpu["pool"].new_empty((33, *cpu["pool"].shape[1:]))
    for step in range(64):
        fresh = torch.randn(case["qkv"].shape, generator=gen).to(torch.bfloat16)
        case["qkv"].copy_(fresh.to(gpu))
        cpu["qkv"].copy_(fresh)
        before = cpu["pool"].clone()
        raw = expected_decode(*[cpu[k] for k in ORDER], 1e-6, return_pre=True)
        packed_reference_step(*[cpu[k] for k in ORDER], 1e-6, scratch=scratch)
        torch.ops.lightdelta.decode(*args_of(case), 1e-6)
        # the indexed restatement and the packed reference path agree bit for bit
        assert torch.equal(raw[0], cpu["out"]) and torch.equal(raw[1], cpu["pool"])
        flips += assert_bf16_outputs(case["out"], cpu["out"], raw[2], label=f"step {step}")["flips"]
        del before
    assert_states(case["pool"], cpu["pool"], label="pool after 64 steps")
    print(f"rounding flips over 64 steps ({policy}): {flips} of {64 * case['out'].numel()}")


def test_mtp_verify_and_commit(gpu):
    """MTP verify at B=64, T=4: each sequence has a base slot and a 4-deep per-token scratch;
    the step reads the base slot, writes the 4 per-token states to the scratch, then
    copy_state commits scratch[accepted-1] to the base slot for a random accepted length."""
    announce(test="mtp_verify_and_commit")
    batch, width = 64, 4
    case = decode_case(batch, width, pool_slots=1 + batch * (width + 1), seed=9, device=gpu)
    ids = torch.randperm(batch * (width + 1), generator=torch.Generator().manual_seed(4)) + 1
    base = ids[:batch].to(torch.int32)
    scratch = ids[batch:].view(batch, width).to(torch.int32)
    # source = base slot: accepted=1 with slots[:, 0] = base, scratch columns hold tokens
    # 1..3; token 0's state goes to the base slot's scratch twin via an explicit column.
    slots = torch.cat([base[:, None], scratch[:, 1:]], 1)
    case["slots"].copy_(slots.to(gpu))
    case["accepted"].fill_(1)
    exp_out, exp_pool, pre = expected(case)
    torch.ops.lightdelta.decode(*args_of(case), 1e-6)
    accept = torch.randint(1, width + 1, (batch,), generator=torch.Generator().manual_seed(8))
    src = slots.gather(1, (accept - 1)[:, None]).flatten().to(torch.int32)
    src[accept == 1] = 0  # accepted length 1: the state already lives in the base slot
    torch.ops.lightdelta.copy_state(case["pool"], src.to(gpu), base.to(gpu))
    torch.cuda.synchronize()
    committed = oracle_state_io.copy(exp_pool.numpy(), src.numpy(), base.numpy())
    assert_bf16_outputs(case["out"], exp_out, pre)
    assert_states(case["pool"], torch.from_numpy(committed), **STEP_STATE)
