"""CPU checks of the host-side logic: the packed Torch path of GDNBackend
(compute="torch_reference") and the oracle's two restatements of the op semantics
(per-request indexed and packed gather/compute/index_copy_) agree on the reference's edge
cases; the numpy state-I/O oracle agrees with element-wise brute force."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lightdelta_amd.backend import GDNBackend
from lightdelta_amd.config import BackendConfig
from lightdelta_amd.workloads import decode_case
from oracle import state_io
from oracle.decode import expected_decode, packed_reference_step

ORDER = ("qkv", "a", "b", "a_log", "dt_bias", "slots", "cu", "accepted", "pool", "gate",
         "weight", "out")


def small_case(batch, width, seed=0, heads=(2, 4)):
    return decode_case(batch, width, num_k_heads=heads[0], num_v_heads=heads[1],
                       pool_slots=batch * width + 2, seed=seed, device="cpu")


def run_three_ways(case, eps=1e-6):
    exp_out, exp_pool = expected_decode(*[case[k] for k in ORDER], eps)
    packed = {k: v.clone() for k, v in case.items()}
    packed_reference_step(*[packed[k] for k in ORDER], eps)
    backend = {k: v.clone() for k, v in case.items()}
    GDNBackend(BackendConfig())(*[backend[k] for k in ORDER], eps)
    return (exp_out, exp_pool), (packed["out"], packed["pool"]), (backend["out"], backend["pool"])


@pytest.mark.parametrize("width", [1, 2, 3, 4])
def test_restatements_agree_with_padding_and_accepted(width):
    case = small_case(4, width, seed=width)
    case["accepted"][:] = torch.arange(4) % width + 1
    case["slots"][-1] = 0
    (eo, ep), (po, pp), (bo, bp) = run_three_ways(case)
    # outputs: identical bits; states: the same math on differently batched tensors
    assert torch.equal(eo, po) and torch.equal(eo, bo)
    torch.testing.assert_close(ep, pp, rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(ep, bp, rtol=1e-6, atol=1e-7)
    assert torch.equal(pp[0], case["pool"][0])


def test_restatements_agree_on_ragged_metadata():
    """cu=[0,4,7,8,8], invalid accepted, a discarded candidate (reference test_gdn.py:105-122)."""
    case = small_case(4, 4, seed=3)
    case["cu"] = torch.tensor([0, 4, 7, 8, 8], dtype=torch.int32)
    case["accepted"][0] = 0
    case["slots"][1, 2] = 0
    for name in ("qkv", "a", "b", "gate", "out"):
        case[name] = case[name][:8]
    (eo, ep), (po, pp), (bo, bp) = run_three_ways(case)
    assert torch.equal(eo, po) and torch.equal(eo, bo)
    torch.testing.assert_close(ep, pp, rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(ep, bp, rtol=1e-6, atol=1e-7)
    assert eo[:4].count_nonzero() == 0


def test_backend_counts_calls():
    case = small_case(2, 1)
    backend = GDNBackend(BackendConfig())
    backend(*[case[k] for k in ORDER])
    case2 = small_case(2, 3)
    backend(*[case2[k] for k in ORDER])
    assert backend.calls == {"decode": 1, "verify": 1}


def test_backend_rejects_invalid_config():
    with pytest.raises(ValueError):
        GDNBackend(BackendConfig(compute="torch_reference", state_io="indexed"))


def test_fused_path_needs_the_hip_library_or_a_device():
    """The fused packed path never falls back to Torch: on CPU tensors it errors."""
    case = small_case(2, 1)
    backend = GDNBackend(BackendConfig(compute="cuda_fused", state_io="packed"))
    with pytest.raises((RuntimeError, NotImplementedError)):
        backend(*[case[k] for k in ORDER])


def _brute_gather(pool, slots, valid):
    out = np.zeros((len(slots),) + pool.shape[1:], pool.dtype)
    for r in range(len(slots)):
        for i in np.ndindex(pool.shape[1:]):
            out[(r,) + i] = pool[(slots[r],) + i] if slots[r] > 0 and valid[r] else 0
    return out


def test_state_io_oracle_against_brute_force():
    rng = np.random.default_rng(1)
    pool = rng.standard_normal((7, 2, 3)).astype(np.float32)
    slots = np.array([3, 0, -1, 6, 3])
    valid = np.array([1, 1, 1, 0, 1], bool)
    assert np.array_equal(state_io.gather(pool, slots, valid), _brute_gather(pool, slots, valid))
    packed = rng.standard_normal((5, 2, 3)).astype(np.float32)
    dst = np.array([1, 0, 2, -1, 5])
    result = state_io.scatter(packed, dst, pool)
    for r, d in enumerate(dst):
        if d > 0:
            assert np.array_equal(result[d], packed[r])
    untouched = [s for s in range(7) if s not in (1, 2, 5)]
    assert np.array_equal(result[untouched], pool[untouched])
    src, dst = np.array([1, 5, -1, 4]), np.array([2, 3, 5, 0])
    copied = state_io.copy(pool, src, dst)
    assert np.array_equal(copied[2], pool[1]) and np.array_equal(copied[3], pool[5])
    assert np.array_equal(copied[[0, 1, 4, 5, 6]], pool[[0, 1, 4, 5, 6]])
    zeroed = state_io.zero(pool, np.array([6, -1, 0, 2]))
    assert not zeroed[[2, 6]].any()
    assert np.array_equal(zeroed[[0, 1, 3, 4, 5]], pool[[0, 1, 3, 4, 5]])
    # zeroing through gather with valid = False and scatter back is the same reset
    via_gather = state_io.scatter(state_io.gather(pool, np.array([6, 2]), np.array([0, 0], bool)),
                                  np.array([6, 2]), pool)
    assert np.array_equal(via_gather, zeroed)


def test_copy_rejects_overlapping_pairs():
    """A chain (1->2, 2->3), a cycle (4->5->6->4) and two writes of one slot (1->0 padding
    aside, 3->7 and 2->7) overlap: every pair involved is rejected and writes nothing; the
    independent pair 8->9 and a self pair 10->10 are applied; a pair with a padding slot
    takes no part in any overlap."""
    rng = np.random.default_rng(3)
    pool = rng.standard_normal((12, 2, 3)).astype(np.float32)
    src = np.array([1, 2, 4, 5, 6, 8, 10, 11, -1])
    dst = np.array([2, 3, 5, 6, 4, 9, 10, -1, 8])
    assert list(state_io.copy_rejected(src, dst)) == [True, True, True, True, True, False,
                                                      False, False, False]
    copied = state_io.copy(pool, src, dst)
    assert np.array_equal(copied[9], pool[8])
    assert np.array_equal(copied[[s for s in range(12) if s != 9]],
                          pool[[s for s in range(12) if s != 9]])
    twice = state_io.copy(pool, np.array([3, 2, 8]), np.array([7, 7, 9]))
    assert np.array_equal(twice[7], pool[7]) and np.array_equal(twice[9], pool[8])


def test_copy_kept_pairs_are_order_independent():
    """On random pair sets (many overlaps), the pairs the rule keeps can be applied one after
    another in any order with the same result, which equals the oracle's; and every
    rejected pair shares a slot with another live pair in a way that makes the order matter
    (its source written, or its destination read or written, by another pair)."""
    rng = np.random.default_rng(4)
    for trial in range(200):
        slots, pairs = 12, int(rng.integers(1, 9))
        pool = rng.standard_normal((slots, 4)).astype(np.float32)
        src = rng.integers(-1, slots, pairs)
        dst = rng.integers(-1, slots, pairs)
        rejected = state_io.copy_rejected(src, dst)
        expected = state_io.copy(pool, src, dst)
        kept = [p for p in range(pairs) if src[p] > 0 and dst[p] > 0 and not rejected[p]]
        for _ in range(3):
            result = pool.copy()
            for p in rng.permutation(kept):
                result[dst[p]] = result[src[p]]
            assert np.array_equal(result, expected), trial
        live = [p for p in range(pairs) if src[p] > 0 and dst[p] > 0]
        for p in live:
            others = [q for q in live if q != p]
            touches = any(dst[q] == src[p] or src[q] == dst[p] or dst[q] == dst[p] for q in others)
            assert touches == bool(rejected[p]), trial


def test_copy_rule_catches_a_dropped_condition(monkeypatch):
    """Planted mistake: an oracle that does not reject two writes of one slot keeps a pair the
    order-independence property then fails on."""
    def lenient(src, dst):
        live = [(s, d) if s > 0 and d > 0 else None for s, d in zip(src, dst)]
        return np.array([pair is not None and any(
            q != p and o is not None and (o[1] == pair[0] or o[0] == pair[1])
            for q, o in enumerate(live)) for p, pair in enumerate(live)])

    monkeypatch.setattr(state_io, "copy_rejected", lenient)
    pool = np.arange(10, dtype=np.float32)[:, None]
    src, dst = np.array([3, 2]), np.array([7, 7])
    results = set()
    for order in ([0, 1], [1, 0]):
        result = pool.copy()
        for p in order:
            if not state_io.copy_rejected(src, dst)[p]:
                result[dst[p]] = result[src[p]]
        results.add(float(result[7, 0]))
    assert len(results) == 2  # the lenient rule leaves the outcome order-dependent
