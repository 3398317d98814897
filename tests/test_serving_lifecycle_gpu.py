"""Requests through the ops in the order a serving layer calls them, one pool throughout:

1. a prefill of three new prompts (70, 130 and 5 tokens; chunked form, 64- or 32-token
   chunks) into their slots;
2. three single-token decode steps on those slots;
3. a 4-token speculative verify per request: the state after token t goes to column t of the
   request's slot row [home, s1, s2, s3], then a random accepted length per request;
4. the next single-token step reads the accepted state through `accepted` (the source is
   column accepted - 1, so no copy commits it) and writes home;
5. the release of one request's slot (`zero_slots`) and its reuse by a new 40-token prompt.

Every call's outputs and the whole pool after it are checked against the oracle. The oracle
runs the same calls on its own pool (never on the kernels' results), so differences would
accumulate over the sequence as they would in serving."""

from __future__ import annotations

import pytest
import torch

from lightdelta_amd import ops
from lightdelta_amd.workloads import decode_case
from oracle import state_io as oracle_state_io
from oracle.decode import expected_decode, expected_prefill
from tests.parity import assert_bf16_outputs, assert_states

pytestmark = pytest.mark.gpu

EPS = 1e-6


class Tokens:
    """Seeded per-token inputs (qkv, a, b, gate), handed out call by call."""

    def __init__(self, rows: int, gpu):
        case = decode_case(rows, 1, pool_slots=16, seed=21, device=gpu)
        self.case = case
        self.next = 0

    def take(self, n: int) -> dict:
        rows = slice(self.next, self.next + n)
        self.next += n
        return {k: self.case[k][rows] for k in ("qkv", "a", "b", "gate")}


def layer(case):
    return case["a_log"], case["dt_bias"]


def check(label, out, exp_out, pre, pool, exp_pool):
    print(f"check: {label}", flush=True)
    assert_bf16_outputs(out, exp_out, pre, label=f"{label}: out")
    assert_states(pool, exp_pool, label=f"{label}: pool")


def prefill(tok, case, pool, ref_pool, slots, has_initial, lengths, label):
    n = sum(lengths)
    t = tok.take(n)
    cu = torch.zeros(len(lengths) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lengths), 0)
    slots_t = torch.tensor(slots, dtype=torch.int32)
    init_t = torch.tensor(has_initial, dtype=torch.bool)
    out = torch.zeros(n, pool.shape[1], 128, dtype=torch.bfloat16, device=pool.device)
    a_log, dt_bias = layer(case)
    args = (t["qkv"], t["a"], t["b"], a_log, dt_bias)
    torch.ops.lightdelta.prefill(*args, slots_t.to(pool.device), init_t.to(pool.device),
                                 cu.to(pool.device), pool, t["gate"], case["weight"], out, EPS)
    torch.cuda.synchronize()
    exp_out, exp_pool, pre = expected_prefill(*args, slots_t, init_t, cu, ref_pool, t["gate"],
                                              case["weight"], out.cpu().zero_(), EPS,
                                              return_pre=True)
    check(label, out, exp_out, pre, pool, exp_pool)
    return exp_pool


def decode(tok, case, pool, ref_pool, indices, accepted, tokens_each, label):
    batch, width = indices.shape
    n = batch * tokens_each
    t = tok.take(n)
    cu = torch.arange(0, n + 1, tokens_each, dtype=torch.int32)
    acc = torch.tensor(accepted, dtype=torch.int32)
    out = torch.zeros(n, pool.shape[1], 128, dtype=torch.bfloat16, device=pool.device)
    a_log, dt_bias = layer(case)
    args = (t["qkv"], t["a"], t["b"], a_log, dt_bias)
    torch.ops.lightdelta.decode(*args, indices.to(pool.device), cu.to(pool.device),
                                acc.to(pool.device), pool, t["gate"], case["weight"], out, EPS)
    torch.cuda.synchronize()
    exp_out, exp_pool, pre = expected_decode(*args, indices, cu, acc, ref_pool, t["gate"],
                                             case["weight"], out.cpu().zero_(), EPS,
                                             return_pre=True)
    check(label, out, exp_out, pre, pool, exp_pool)
    return exp_pool


@pytest.mark.parametrize("form", ["chunked", "chunked_32"])
def test_request_lifecycle(gpu, form):
    print(f"case: serving lifecycle, 16/32 heads, 16-slot pool, {form} prefill", flush=True)
    tok = Tokens(70 + 130 + 5 + 3 * 3 + 3 * 4 + 3 + 40, gpu)
    case = tok.case
    pool = case["pool"]
    ref_pool = pool.cpu().clone()
    home = [3, 7, 9]
    scratch = torch.tensor([[1, 2, 4], [5, 6, 8], [10, 11, 12]], dtype=torch.int32)
    saved = ops.prefill_algorithm()
    ops.set_prefill_algorithm(form)
    try:
        ref_pool = prefill(tok, case, pool, ref_pool, home, [False] * 3, [70, 130, 5],
                           "prefill of 3 prompts")
    finally:
        ops.set_prefill_algorithm(saved)
    rows = torch.tensor(home, dtype=torch.int32)[:, None]
    for step in range(3):
        ref_pool = decode(tok, case, pool, ref_pool, rows, [1, 1, 1], 1, f"decode step {step}")
    verify_rows = torch.cat([rows, scratch], 1)
    ref_pool = decode(tok, case, pool, ref_pool, verify_rows, [1, 1, 1], 4, "4-token verify")
    accepted = torch.randint(1, 5, (3,), generator=torch.Generator().manual_seed(5)).tolist()
    print(f"accepted lengths {accepted}", flush=True)
    ref_pool = decode(tok, case, pool, ref_pool, verify_rows, accepted, 1,
                      "step after the verify")
    freed = torch.tensor([home[1]], dtype=torch.int32)
    torch.ops.lightdelta.zero_slots(pool, freed.to(pool.device))
    torch.cuda.synchronize()
    ref_pool = torch.from_numpy(oracle_state_io.zero(ref_pool.numpy(), freed.numpy()))
    assert_states(pool, ref_pool, label="pool after zero_slots")
    ref_pool = prefill(tok, case, pool, ref_pool, [home[1]], [True], [40],
                       "prefill of a new prompt into the freed slot")
