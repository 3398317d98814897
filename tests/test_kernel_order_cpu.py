"""The reference CUDA kernel's summation order (oracle/kernel_order.py) against the reference's
Torch path (oracle/gdn.py), on the CPU.

What it shows: a correct kernel that sums in the reference kernel's own order (32 lanes of 4
consecutive k, fused multiply-adds, an xor butterfly) on the very inputs the Torch path sees
cannot meet rtol = atol = 2e-3 on every bf16 output -- a few outputs land on the other side
of a bf16 rounding -- and every such output is one the parity rule (tests/parity.py) excuses.
The GPU tests hold this build's kernels to the same rule."""

from __future__ import annotations

import torch

from lightdelta_amd.workloads import decode_case
from oracle import kernel_order
from oracle.decode import expected_decode, geometry, split_tokens
from tests.parity import ATOL, RTOL, assert_bf16_outputs, assert_states

ORDER = ("qkv", "a", "b", "a_log", "dt_bias", "slots", "cu", "accepted", "pool", "gate",
         "weight", "out")


def integer_rows(seed: int, rows: int = 64) -> tuple[torch.Tensor, torch.Tensor]:
    gen = torch.Generator().manual_seed(seed)
    h = torch.randint(-8, 9, (rows, 128), generator=gen).float()
    x = torch.randint(-8, 9, (rows, 128), generator=gen).float()
    return h, x


def test_lane_dot_is_the_exact_sum_on_integers():
    """Small integers keep every product and partial sum exact in fp32, so any order gives
    the exact dot product: the lane split and the butterfly cover all 128 terms once."""
    h, x = integer_rows(0)
    got = kernel_order.lane_dot(h, x)
    assert torch.equal(got, (h.double() * x.double()).sum(-1).float())


def test_planted_butterfly_mistake_is_caught():
    """A butterfly without its last stage sums 16 of the 32 lanes: the exact-sum check above
    fails for it."""
    h, x = integer_rows(1)
    wrong = kernel_order.lane_dot(h, x, offsets=(16, 8, 4, 2))
    assert not torch.equal(wrong, (h.double() * x.double()).sum(-1).float())


def test_reference_order_flips_bf16_roundings_at_the_workload_shape():
    """B = 32, 16 qk / 32 v heads, 16 in-place steps (the GPU workload test's inputs): the
    kernel-order trajectory against the Torch path's.  Some outputs miss 2e-3 by a bf16
    rounding, all of them excused as rounding-sensitive, and the states agree to 2e-3."""
    case = decode_case(32, 1, pool_slots=256, seed=0, device="cpu")
    kernel_pool = case["pool"].clone()
    slots = case["slots"][:, 0].long()
    h, hv = geometry(case["qkv"], case["pool"])
    gen = torch.Generator().manual_seed(11)
    strict = flips = 0
    for step in range(16):
        case["qkv"].copy_(torch.randn(case["qkv"].shape, generator=gen).to(torch.bfloat16))
        exp_out, exp_pool, pre = expected_decode(*[case[k] for k in ORDER], 1e-6,
                                                 return_pre=True)
        case["pool"].copy_(exp_pool)
        q, k, v, a, b, gate = (t.transpose(0, 1) for t in split_tokens(
            case["qkv"], case["a"], case["b"], case["gate"], slice(0, 32), h, hv))
        out, state = kernel_order.run_steps(q, k, v, a, b, case["a_log"], case["dt_bias"],
                                            gate, case["weight"], kernel_pool[slots], 1e-6)
        kernel_pool[slots] = state
        got = out[:, 0].float()
        strict += int(((got - exp_out.float()).abs() > ATOL + RTOL * exp_out.float().abs()).sum())
        flips += assert_bf16_outputs(out[:, 0], exp_out, pre, label=f"step {step}")["flips"]
    assert_states(kernel_pool, case["pool"], label="pool after 16 steps")
    print(f"reference kernel order: {strict} outputs outside 2e-3 over 16 steps, "
          f"{flips} excused as rounding flips, of {16 * case['out'].numel()}")
    assert strict > 0, "the reference kernel's order met 2e-3 everywhere on these inputs"
    assert flips == strict
