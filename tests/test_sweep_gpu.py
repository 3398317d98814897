"""Seeded sweeps over random shapes and metadata, against the oracle: the decode step, the
conv-fused step and the prefill, each case drawn from its seed (head layout, batch, width,
ragged token counts, padding slots, out-of-range accepted counts, weight dtypes, cache
policy, conv-state length and layout, prefill algorithm).  The fixed-shape tests cover each
rule on purpose; these cover their combinations.  Positive slot ids are distinct within a
launch (requests never share a slot), as a serving batch's are."""

from __future__ import annotations

import pytest
import torch

from lightdelta_amd import ops
from lightdelta_amd.backend import GDNBackend
from lightdelta_amd.config import BackendConfig
from lightdelta_amd.workloads import decode_case
from oracle.decode import expected_decode, expected_decode_conv, expected_prefill
from tests.parity import assert_bf16_outputs, assert_states

pytestmark = pytest.mark.gpu

HEADS = [(16, 32), (16, 48), (8, 16), (4, 8), (8, 8), (2, 6), (1, 4)]
ORDER = ("qkv", "a", "b", "a_log", "dt_bias", "slots", "cu", "accepted", "pool", "gate",
         "weight", "out")
PREFILL = ("qkv", "a", "b", "a_log", "dt_bias", "slots", "has_initial", "cu_seqlens", "pool",
           "gate", "weight", "out")
# The reference's one-step state tolerance (tests/test_gdn.py:74).
STEP_STATE = dict(rtol=3e-4, atol=3e-6)


class Draw:
    """Integers and choices from one seeded generator."""

    def __init__(self, seed: int):
        self.gen = torch.Generator().manual_seed(seed)

    def int(self, lo: int, hi: int) -> int:  # inclusive
        return int(torch.randint(lo, hi + 1, (1,), generator=self.gen))

    def pick(self, items):
        return items[self.int(0, len(items) - 1)]


@pytest.fixture
def restore_settings():
    policy, algorithm = ops.state_cache_policy(), ops.prefill_algorithm()
    yield
    ops.set_state_cache_policy(policy)
    ops.set_prefill_algorithm(algorithm)


def padded_slots(d: Draw, count: int, pool_slots: int) -> torch.Tensor:
    """`count` distinct slot ids in [1, pool_slots), about one in seven replaced by a padding
    id (0 or -1)."""
    ids = torch.randperm(pool_slots - 1, generator=d.gen)[:count] + 1
    pad = torch.rand(count, generator=d.gen) < 0.15
    fill = torch.where(torch.rand(count, generator=d.gen) < 0.5, 0, -1)
    return torch.where(pad, fill, ids).to(torch.int32)


def random_step_case(gpu, seed: int, conv: bool = False, longer: bool = True):
    """A decode (or conv-fused decode) launch drawn from `seed`: returns (case, cache policy,
    description).  `longer`: sometimes one request with more tokens than its width."""
    d = Draw(seed)
    h, hv = d.pick(HEADS)
    batch, width = d.int(1, 40), d.int(1, 4)
    lengths = torch.randint(0, width + 1, (batch,), generator=d.gen)
    if longer and not conv and d.int(0, 3) == 0:  # a request longer than its width: rejected
        lengths[d.int(0, batch - 1)] = width + 1
    tokens = int(lengths.sum())
    pool_slots = batch * width + 3
    dt_dtype = d.pick([torch.float32, torch.bfloat16])
    w_dtype = d.pick([torch.float32, torch.bfloat16])
    case = decode_case(max(tokens, 1), 1, num_k_heads=h, num_v_heads=hv, pool_slots=pool_slots,
                       seed=seed, device=gpu, dt_bias_dtype=dt_dtype, weight_dtype=w_dtype)
    for name in ("qkv", "a", "b", "gate", "out"):
        case[name] = case[name][:tokens]
    cu = torch.zeros(batch + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lengths, 0)
    case["cu"] = cu.to(gpu)
    case["slots"] = padded_slots(d, batch * width, pool_slots).view(batch, width).to(gpu)
    case["accepted"] = torch.randint(-1, width + 2, (batch,), generator=d.gen,
                                     dtype=torch.int32).to(gpu)
    policy = d.pick(["keep", "stream"])
    what = dict(seed=seed, heads=(h, hv), batch=batch, width=width, tokens=tokens,
                dt=str(dt_dtype)[6:], w=str(w_dtype)[6:], policy=policy)
    if conv:
        conv_dim = case["qkv"].shape[1] if tokens else (2 * h + hv) * 128
        length = d.int(3, 8) if width > 1 else d.pick([3, 4, 3 + d.int(0, 5)])
        length = max(length, 3 + width - 1)  # the state holds a speculative step's history
        dim_last = d.int(0, 1) == 1
        bias = d.int(0, 1) == 1
        if dim_last:
            conv_state = torch.randn(pool_slots, length, conv_dim, generator=d.gen
                                     ).bfloat16().to(gpu).transpose(1, 2)
        else:
            conv_state = torch.randn(pool_slots, conv_dim, length, generator=d.gen
                                     ).bfloat16().to(gpu)
        case["conv_state"] = conv_state
        case["conv_weight"] = (torch.randn(conv_dim, 4, generator=d.gen) / 2).bfloat16().to(gpu)
        case["conv_bias"] = (torch.randn(conv_dim, generator=d.gen).bfloat16().to(gpu)
                             if bias else None)
        what.update(conv_len=length, dim_last=dim_last, bias=bias)
    return case, policy, what


def announce(what: dict) -> None:
    print("case:", " ".join(f"{k}={v}" for k, v in what.items()), flush=True)


@pytest.mark.parametrize("seed", range(40))
def test_decode_sweep(gpu, seed, restore_settings):
    case, policy, what = random_step_case(gpu, seed)
    announce(dict(test="decode_sweep", **what))
    ops.set_state_cache_policy(policy)
    args = [case[k] for k in ORDER]
    exp_out, exp_pool, pre = expected_decode(*args, 1e-6, return_pre=True)
    before = case["pool"].clone()
    torch.ops.lightdelta.decode(*args, 1e-6)
    torch.cuda.synchronize()
    assert_bf16_outputs(case["out"], exp_out, pre, label=f"seed {seed}")
    assert_states(case["pool"], exp_pool, label=f"seed {seed}", **STEP_STATE)
    assert torch.equal(case["pool"][0], before[0])


@pytest.mark.parametrize("seed", range(300, 320))
def test_backend_packed_sweep(gpu, seed, restore_settings):
    """GDNBackend's packed path (packed_plan, gather_state, the step on the scratch,
    scatter_state) on the same draws, token counts within the width (device metadata the
    backend trusts, as the reference's does)."""
    case, policy, what = random_step_case(gpu, seed, longer=False)
    announce(dict(test="backend_packed_sweep", **what))
    ops.set_state_cache_policy(policy)
    args = [case[k] for k in ORDER]
    exp_out, exp_pool, pre = expected_decode(*args, 1e-6, return_pre=True)
    before = case["pool"].clone()
    GDNBackend(BackendConfig(compute="cuda_fused", state_io="packed"))(*args, 1e-6)
    torch.cuda.synchronize()
    assert_bf16_outputs(case["out"], exp_out, pre, label=f"seed {seed}")
    assert_states(case["pool"], exp_pool, label=f"seed {seed}", **STEP_STATE)
    assert torch.equal(case["pool"][0], before[0])


@pytest.mark.parametrize("seed", range(100, 130))
def test_decode_conv_sweep(gpu, seed, restore_settings):
    case, policy, what = random_step_case(gpu, seed, conv=True)
    announce(dict(test="decode_conv_sweep", **what))
    ops.set_state_cache_policy(policy)
    rest = [case[k] for k in ORDER[1:]]
    exp_out, exp_pool, pre, exp_conv, _ = expected_decode_conv(
        case["qkv"], case["conv_state"], case["conv_weight"], case["conv_bias"], *rest, 1e-6,
        return_pre=True)
    torch.ops.lightdelta.decode_conv(case["qkv"], case["conv_state"], case["conv_weight"],
                                     case["conv_bias"], *rest, 1e-6)
    torch.cuda.synchronize()
    got_conv = case["conv_state"].cpu()
    if not torch.equal(got_conv, exp_conv):
        bad = (got_conv != exp_conv).nonzero()
        raise AssertionError(f"seed {seed}: conv state differs at {len(bad)} elements "
                             f"(slot, channel, column), first {bad[:6].tolist()}")
    assert_bf16_outputs(case["out"], exp_out, pre, label=f"seed {seed}")
    assert_states(case["pool"], exp_pool, label=f"seed {seed}", **STEP_STATE)


@pytest.mark.parametrize("seed", range(200, 224))
def test_prefill_sweep(gpu, seed, restore_settings):
    d = Draw(seed)
    h, hv = d.pick(HEADS)
    count = d.int(1, 24)
    long_prompts = d.int(0, 2) == 0
    lengths = torch.randint(0, 300 if long_prompts else 48, (count,), generator=d.gen)
    algorithm = d.pick(["auto", "token_serial", "chunked", "chunked_32"])
    dt_dtype = d.pick([torch.float32, torch.bfloat16])
    w_dtype = d.pick([torch.float32, torch.bfloat16])
    tokens = int(lengths.sum())
    pool_slots = count + 3
    announce(dict(test="prefill_sweep", seed=seed, heads=(h, hv), sequences=count,
                  tokens=tokens, algorithm=algorithm))
    case = decode_case(max(tokens, 1), 1, num_k_heads=h, num_v_heads=hv, pool_slots=pool_slots,
                       seed=seed, device=gpu, dt_bias_dtype=dt_dtype, weight_dtype=w_dtype)
    for name in ("qkv", "a", "b", "gate", "out"):
        case[name] = case[name][:tokens]
    case["slots"] = padded_slots(d, count, pool_slots).to(gpu)
    case["has_initial"] = (torch.rand(count, generator=d.gen) < 0.6).to(gpu)
    cu = torch.zeros(count + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lengths, 0)
    case["cu_seqlens"] = cu.to(gpu)
    ops.set_prefill_algorithm(algorithm)
    args = [case[k] for k in PREFILL]
    exp_out, exp_pool, pre = expected_prefill(*args, 1e-6, return_pre=True)
    before = case["pool"].clone()
    torch.ops.lightdelta.prefill(*args, 1e-6)
    torch.cuda.synchronize()
    assert_bf16_outputs(case["out"], exp_out, pre, label=f"seed {seed}")
    assert_states(case["pool"], exp_pool, label=f"seed {seed}")
    assert torch.equal(case["pool"][0], before[0])
