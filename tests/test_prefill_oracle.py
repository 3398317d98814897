"""The prefill oracle (oracle/decode.py expected_prefill) against the reference's own
vectors: tests/golden/cfg1_64.npz holds 64 consecutive steps of the reference's
post_conv_gdn on one sequence (4 qk / 8 v heads), which is the prefill of those 64 tokens
from the same initial state.  Also the layer's slot semantics: padding, has_initial, empty
sequences, and sequences independent of their neighbours."""

from __future__ import annotations

import torch

from lightdelta_amd.workloads import decode_case
from oracle.decode import expected_prefill
from tests.conftest import load_golden


def pack_golden(g):
    """The golden q/k/v/gate/a/b of one sequence as the op's packed row layout."""
    q, k, v = g["q"][0], g["k"][0], g["v"][0]  # [T, H, 128] / [T, HV, 128]
    tokens = q.shape[0]
    qkv = torch.cat([q.reshape(tokens, -1), k.reshape(tokens, -1), v.reshape(tokens, -1)], 1)
    return qkv, g["a"][0], g["b"][0], g["gate"][0]


def test_prefill_of_64_tokens_matches_the_reference_steps():
    g = load_golden("cfg1_64")
    qkv, a, b, gate = pack_golden(g)
    pool = torch.zeros(3, *g["state"].shape[1:])
    pool[2] = g["state"][0]
    out = torch.zeros(qkv.shape[0], 8, 128, dtype=torch.bfloat16)
    new_out, new_pool = expected_prefill(
        qkv, a, b, g["a_log"], g["dt_bias"], torch.tensor([2], dtype=torch.int32),
        torch.tensor([True]), torch.tensor([0, 64], dtype=torch.int32), pool, gate,
        g["norm_weight"], out, 1e-6)
    # one 64-token call vs 64 one-token calls of the reference: the same per-token
    # arithmetic, up to the reduction order of the vectorised L2 norms
    diff = (new_out.float() - g["output"][0].float()).abs()
    assert diff.max() <= 2**-9 and int((diff > 0).sum()) <= 16  # measured: 4 of 65536, 1 ulp
    torch.testing.assert_close(new_pool[2], g["final_state"][0], rtol=1e-5, atol=1e-6)
    assert torch.equal(new_pool[0], pool[0]) and torch.equal(new_pool[1], pool[1])


def test_slot_semantics_and_independence():
    case = decode_case(4, 1, num_k_heads=4, num_v_heads=8, pool_slots=6, seed=3, device="cpu")
    rows = case["qkv"].shape[0]
    args = lambda slots, init, cu, pool: (  # noqa: E731
        case["qkv"], case["a"], case["b"], case["a_log"], case["dt_bias"], slots, init, cu, pool,
        case["gate"], case["weight"], torch.zeros(rows, 8, 128, dtype=torch.bfloat16), 1e-6)
    pool = case["pool"]
    slots = torch.tensor([3, 0, 5], dtype=torch.int32)
    init = torch.tensor([True, True, False])
    cu = torch.tensor([0, 2, 2, 4], dtype=torch.int32)  # second sequence empty
    out, new_pool = expected_prefill(*args(slots, init, cu, pool))
    assert torch.equal(new_pool[0], pool[0])  # padding slot: never written
    assert new_pool[5].abs().sum() > 0 and not torch.equal(new_pool[5], pool[5])
    # has_initial False == a zero initial state
    zeroed = pool.clone()
    zeroed[5] = 0
    out_z, pool_z = expected_prefill(*args(slots, torch.tensor([True, True, True]), cu, zeroed))
    assert torch.equal(out, out_z) and torch.equal(new_pool[5], pool_z[5])
    # a sequence alone gives the same result as inside the batch
    out1, pool1 = expected_prefill(*args(slots[:1], init[:1], cu[:2], pool))
    assert torch.equal(out1[:2], out[:2]) and torch.equal(pool1[3], new_pool[3])
    # an empty sequence with has_initial writes its initial state back unchanged
    out_e, pool_e = expected_prefill(*args(torch.tensor([4], dtype=torch.int32),
                                           torch.tensor([True]), torch.tensor([0, 0], dtype=torch.int32),
                                           pool))
    assert torch.equal(pool_e, pool)
