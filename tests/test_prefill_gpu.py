"""Parity of the gfx950 prefill (torch.ops.lightdelta.prefill) with the oracle's restatement
of the layer's prefill (oracle/decode.py expected_prefill), under every algorithm
(token-serial, and 64- or 32-token chunks in the WY form); and, for the token-serial one, with
the decode kernel: a prefill of n tokens must give bit for bit the states and outputs of n
single-token decode steps on the same slot (the per-token arithmetic is shared)."""

from __future__ import annotations

import pytest
import torch

from lightdelta_amd import _lib, ops
from lightdelta_amd.workloads import decode_case
from oracle.decode import expected_prefill
from tests.parity import assert_bf16_outputs, assert_states

pytestmark = pytest.mark.gpu

PREFILL = ("qkv", "a", "b", "a_log", "dt_bias", "slots", "has_initial", "cu_seqlens", "pool",
           "gate", "weight", "out")


def announce(**what):
    print("case:", " ".join(f"{k}={v}" for k, v in what.items()), flush=True)


def prefill_case(gpu, lengths, heads=(16, 32), pool_slots=None, seed=0, dt_dtype=torch.float32,
                 w_dtype=torch.float32):
    """Sequences of the given lengths packed row after row; one slot per sequence."""
    total = sum(lengths)
    n = len(lengths)
    pool_slots = pool_slots or n + 2
    case = decode_case(max(total, 1), 1, num_k_heads=heads[0], num_v_heads=heads[1],
                       pool_slots=pool_slots, seed=seed, device=gpu,
                       dt_bias_dtype=dt_dtype, weight_dtype=w_dtype)
    for name in ("qkv", "a", "b", "gate", "out"):
        case[name] = case[name][:total]
    gen = torch.Generator().manual_seed(seed + 1)
    case["slots"] = (torch.randperm(case["pool"].shape[0] - 1, generator=gen)[:n] + 1).to(
        torch.int32).to(gpu)
    case["has_initial"] = torch.ones(n, dtype=torch.bool, device=gpu)
    cu = torch.zeros(n + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lengths), 0)
    case["cu_seqlens"] = cu.to(gpu)
    return case


def run(case, eps=1e-6):
    torch.ops.lightdelta.prefill(*[case[k] for k in PREFILL], eps)


CHUNKED_FORMS = ["chunked", "chunked_32"]


@pytest.fixture(params=["token_serial", *CHUNKED_FORMS])
def algorithm(request):
    saved = ops.prefill_algorithm()
    ops.set_prefill_algorithm(request.param)
    yield request.param
    ops.set_prefill_algorithm(saved)


@pytest.fixture
def token_serial():
    saved = ops.prefill_algorithm()
    ops.set_prefill_algorithm("token_serial")
    yield
    ops.set_prefill_algorithm(saved)


@pytest.mark.parametrize("heads", [(16, 32), (4, 8), (16, 48), (8, 8)])
def test_prefill_matches_oracle(gpu, heads, algorithm):
    announce(test="prefill_oracle", heads=heads, algorithm=algorithm)
    case = prefill_case(gpu, [5, 0, 1, 33, 70], heads=heads, seed=heads[1])
    case["has_initial"][3] = False  # starts from zeros
    case["slots"][2] = 0  # padding slot: zero initial state, final state dropped
    exp_out, exp_pool, pre = expected_prefill(*[case[k] for k in PREFILL], 1e-6, return_pre=True)
    before = case["pool"].clone()
    run(case)
    torch.cuda.synchronize()
    assert_bf16_outputs(case["out"], exp_out, pre)
    assert_states(case["pool"], exp_pool)
    assert torch.equal(case["pool"][0], before[0])


@pytest.mark.parametrize("heads", [(16, 32), (4, 8), (16, 48), (8, 8)])
@pytest.mark.parametrize("form", CHUNKED_FORMS)
def test_prefill_longer_prompts_match_oracle(gpu, heads, form):
    """Prompts of 40 tokens or more on average (the 32-token form's split products, several
    chunks per prompt), every head layout, against the oracle."""
    announce(test="prefill_oracle_longer", heads=heads, form=form)
    saved = ops.prefill_algorithm()
    ops.set_prefill_algorithm(form)
    try:
        case = prefill_case(gpu, [40, 0, 97, 33, 65], heads=heads, seed=heads[1] + 1)
        case["has_initial"][2] = False
        case["slots"][4] = 0  # padding slot
        exp_out, exp_pool, pre = expected_prefill(*[case[k] for k in PREFILL], 1e-6,
                                                  return_pre=True)
        run(case)
        torch.cuda.synchronize()
    finally:
        ops.set_prefill_algorithm(saved)
    assert_bf16_outputs(case["out"], exp_out, pre)
    assert_states(case["pool"], exp_pool)


@pytest.mark.parametrize("dt_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("w_dtype", [torch.float32, torch.bfloat16])
def test_prefill_parameter_dtypes(gpu, dt_dtype, w_dtype, algorithm):
    announce(test="prefill_dtypes", dt=dt_dtype, w=w_dtype, algorithm=algorithm)
    case = prefill_case(gpu, [9, 17], seed=2, dt_dtype=dt_dtype, w_dtype=w_dtype)
    exp_out, exp_pool, pre = expected_prefill(*[case[k] for k in PREFILL], 1e-6, return_pre=True)
    run(case)
    torch.cuda.synchronize()
    assert_bf16_outputs(case["out"], exp_out, pre)
    assert_states(case["pool"], exp_pool)


def decode_steps(case, eps=1e-6):
    """The same sequences as single-token decode steps, one launch per token, on a copy of
    the pool; returns (out, pool)."""
    pool = case["pool"].clone()
    out = torch.zeros_like(case["out"])
    cu = case["cu_seqlens"].cpu().tolist()
    one = torch.ones(1, dtype=torch.int32, device=pool.device)
    for n, slot in enumerate(case["slots"].cpu().tolist()):
        if not bool(case["has_initial"][n]):
            pool[slot].zero_()
        for t in range(cu[n], cu[n + 1]):
            torch.ops.lightdelta.decode(
                case["qkv"][t:t + 1], case["a"][t:t + 1], case["b"][t:t + 1], case["a_log"],
                case["dt_bias"], case["slots"][n:n + 1].view(1, 1),
                torch.tensor([0, 1], dtype=torch.int32, device=pool.device), one, pool,
                case["gate"][t:t + 1], case["weight"], out[t:t + 1], eps)
    return out, pool


def test_prefill_equals_decode_steps_bit_for_bit(gpu, token_serial):
    announce(test="prefill_vs_decode")
    case = prefill_case(gpu, [3, 40, 1, 77], seed=5)
    case["has_initial"][1] = False
    exp_out, exp_pool = decode_steps(case)
    run(case)
    torch.cuda.synchronize()
    assert torch.equal(case["out"], exp_out)
    assert torch.equal(case["pool"], exp_pool)


def test_long_prompt(gpu, token_serial):
    """One 2048-token prompt at 16/32 heads: bit-exact against 2048 decode steps, and within
    the build's tolerance of the oracle's state after 2048 recurrent steps."""
    announce(test="prefill_long")
    case = prefill_case(gpu, [2048], seed=6)
    exp_out, exp_pool = decode_steps(case)
    oracle_out, oracle_pool = expected_prefill(*[case[k] for k in PREFILL], 1e-6)
    run(case)
    torch.cuda.synchronize()
    assert torch.equal(case["out"], exp_out)
    assert torch.equal(case["pool"], exp_pool)
    assert_states(case["pool"], oracle_pool)
    torch.testing.assert_close(case["out"].float().cpu(), oracle_out.float(), atol=8e-3, rtol=2e-2)


def test_prefill_graph_capture(gpu, algorithm):
    announce(test="prefill_graph", algorithm=algorithm)
    case = prefill_case(gpu, [12, 30, 7], seed=8)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run(case)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(case)
    gen = torch.Generator().manual_seed(9)
    for replay in range(3):
        case["slots"].copy_((torch.randperm(case["pool"].shape[0] - 1, generator=gen)[:3] + 1)
                            .to(torch.int32))
        exp_out, exp_pool, pre = expected_prefill(*[case[k] for k in PREFILL], 1e-6,
                                                  return_pre=True)
        graph.replay()
        torch.cuda.synchronize()
        assert_bf16_outputs(case["out"], exp_out, pre, label=f"replay {replay}")
        assert_states(case["pool"], exp_pool, label=f"replay {replay}")


def test_captured_chunked_workspace_outlives_the_eager_cache(gpu):
    """The chunked form under graph capture on a stream whose eager workspace is cached: after
    the capture, a larger eager prefill on that stream (which replaces the cached buffer) and
    release_prefill_workspaces() (which drops it), new tensors of the freed sizes are
    allocated on that stream and filled; the replays must still match the oracle and leave those tensors
    untouched (the graph's workspace is its own, not the cache's)."""
    announce(test="prefill_graph_workspace")
    saved = ops.prefill_algorithm()
    ops.set_prefill_algorithm("chunked")
    try:
        case = prefill_case(gpu, [100, 70], seed=11)
        big = prefill_case(gpu, [300, 260, 200], seed=12)
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            run(case)  # eager: caches a workspace for this stream
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            run(case)
        with torch.cuda.stream(stream):
            run(big)  # eager, larger: the cached buffer is replaced
        torch.cuda.synchronize()
        ops.release_prefill_workspaces()
        lib = _lib.load()
        sizes = [lib.ld_gdn_prefill_workspace_bytes(170, 2, 32)] * 4 + \
            [lib.ld_gdn_prefill_workspace_bytes(760, 3, 32)] * 2
        with torch.cuda.stream(stream):  # the allocator reuses a stream's own freed blocks
            fillers = [torch.full((n,), 0x5A, dtype=torch.uint8, device=gpu) for n in sizes]
        torch.cuda.synchronize()
        gen = torch.Generator().manual_seed(13)
        for replay in range(3):
            case["slots"].copy_((torch.randperm(case["pool"].shape[0] - 1, generator=gen)[:2] + 1)
                                .to(torch.int32))
            exp_out, exp_pool, pre = expected_prefill(*[case[k] for k in PREFILL], 1e-6,
                                                      return_pre=True)
            graph.replay()
            torch.cuda.synchronize()
            assert_bf16_outputs(case["out"], exp_out, pre, label=f"replay {replay}")
            assert_states(case["pool"], exp_pool, label=f"replay {replay}")
            for i, f in enumerate(fillers):
                assert bool((f == 0x5A).all()), f"replay {replay}: filler {i} was overwritten"
    finally:
        ops.set_prefill_algorithm(saved)


@pytest.mark.parametrize("sequences", [16, 32])
def test_split_and_fused_paths_agree(gpu, sequences, token_serial):
    """32 sequences x 32 heads fill the GPU (one workgroup per head, fused norm); 16 split each
    head's rows in two; one sequence alone splits them in four with the norm as a second
    launch.  All must give the same bits, and match the oracle."""
    announce(test="prefill_paths", sequences=sequences)
    gen = torch.Generator().manual_seed(sequences)
    lengths = torch.randint(0, 24, (sequences,), generator=gen).tolist()
    case = prefill_case(gpu, lengths, seed=sequences, pool_slots=sequences + 2)
    case["has_initial"][::3] = False
    exp_out, exp_pool, pre = expected_prefill(*[case[k] for k in PREFILL], 1e-6, return_pre=True)
    pool0 = case["pool"].clone()
    run(case)
    torch.cuda.synchronize()
    assert_bf16_outputs(case["out"], exp_out, pre)
    assert_states(case["pool"], exp_pool)
    batch_out, batch_pool = case["out"].clone(), case["pool"].clone()
    case["pool"].copy_(pool0)
    case["out"].zero_()
    cu = case["cu_seqlens"]
    for n in range(sequences):
        one = dict(case)
        one["slots"] = case["slots"][n:n + 1]
        one["has_initial"] = case["has_initial"][n:n + 1]
        one["cu_seqlens"] = cu[n:n + 2]
        run(one)
    torch.cuda.synchronize()
    assert torch.equal(case["out"], batch_out)
    assert torch.equal(case["pool"], batch_pool)


def chunked_against_token_serial(case, form):
    """Runs `case` under the token-serial and the chunked form `form` from the same pool;
    checks the chunked results within the build's tolerance of the token-serial ones."""
    pool0 = case["pool"].clone()
    saved = ops.prefill_algorithm()
    try:
        ops.set_prefill_algorithm("token_serial")
        run(case)
        torch.cuda.synchronize()
        ref_out, ref_pool = case["out"].clone(), case["pool"].clone()
        case["pool"].copy_(pool0)
        case["out"].zero_()
        ops.set_prefill_algorithm(form)
        run(case)
        torch.cuda.synchronize()
    finally:
        ops.set_prefill_algorithm(saved)
    assert_states(case["pool"], ref_pool)
    torch.testing.assert_close(case["out"].float(), ref_out.float(), atol=8e-3, rtol=2e-2)
    close = ((case["out"].float() - ref_out.float()).abs() <= 2e-3 + 2e-3 * ref_out.float().abs())
    assert close.float().mean() > 0.999


@pytest.mark.parametrize("form", CHUNKED_FORMS)
def test_chunked_long_prompts_match_the_token_serial_form(gpu, form):
    """Two prompts of 1000 and 3000 tokens (partial last chunks) under the chunked form:
    within the build's tolerance of the token-serial results after thousands of steps."""
    announce(test="prefill_chunked_long", form=form)
    case = prefill_case(gpu, [1000, 3000], seed=11)
    case["has_initial"][0] = False
    chunked_against_token_serial(case, form)


@pytest.mark.parametrize("form", CHUNKED_FORMS)
def test_chunked_two_row_tiles_over_many_chunks(gpu, form):
    """16 prompts of 200 to 330 tokens (partial last chunks), 16 qk / 32 v heads: 512
    (sequence, head) pairs, so the scan takes two 16-row state tiles per workgroup with one
    operand set refilled half a chunk ahead, over several chunks per sequence."""
    announce(test="prefill_chunked_two_row_tiles", form=form)
    gen = torch.Generator().manual_seed(15)
    lengths = torch.randint(200, 331, (16,), generator=gen).tolist()
    case = prefill_case(gpu, lengths, seed=15)
    case["has_initial"][1::3] = False
    chunked_against_token_serial(case, form)


@pytest.mark.parametrize("form", CHUNKED_FORMS)
def test_chunked_many_sequences_match_the_token_serial_form(gpu, form):
    """300 sequences of 0 to 150 tokens (empty ones among them; more sequences than one round
    of the chunk-index scan covers), some from zero states, one on the padding slot."""
    announce(test="prefill_chunked_many", form=form)
    gen = torch.Generator().manual_seed(12)
    lengths = torch.randint(0, 151, (300,), generator=gen).tolist()
    lengths[0] = lengths[150] = lengths[299] = 0
    lengths[256] = 64
    case = prefill_case(gpu, lengths, seed=12)
    case["has_initial"][::7] = False
    case["slots"][3] = 0
    chunked_against_token_serial(case, form)


@pytest.mark.parametrize("form", CHUNKED_FORMS)
def test_chunked_short_prompts_match_the_token_serial_form(gpu, form):
    """1024 prompts of 1 to 48 tokens (one or two 32-token chunks each, a part of one 64-token
    chunk), the shapes the 32-token form is for; some from zero states."""
    announce(test="prefill_chunked_short", form=form)
    gen = torch.Generator().manual_seed(31)
    lengths = torch.randint(1, 49, (1024,), generator=gen).tolist()
    lengths[5], lengths[6], lengths[7] = 32, 33, 31
    case = prefill_case(gpu, lengths, seed=31)
    case["has_initial"][::5] = False
    chunked_against_token_serial(case, form)


@pytest.mark.parametrize("form", CHUNKED_FORMS)
@pytest.mark.parametrize("layout", ["odd_row_stride", "shifted_base"])
def test_chunked_unaligned_rows_match_aligned_rows(gpu, layout, form):
    """qkv rows that do not start at 16-byte boundaries (an odd row stride, or a base one
    element past one) take the chunked prep's one- and two-element loads instead of its
    16-byte pieces: the same values and arithmetic, so the same bits."""
    announce(test="prefill_chunked_unaligned", layout=layout, form=form)
    case = prefill_case(gpu, [130, 64, 7, 200, 0, 65], seed=21)
    case["has_initial"][1] = False
    pool0 = case["pool"].clone()
    saved = ops.prefill_algorithm()
    ops.set_prefill_algorithm(form)
    try:
        run(case)
        torch.cuda.synchronize()
        ref_out, ref_pool = case["out"].clone(), case["pool"].clone()
        n, cols = case["qkv"].shape
        if layout == "odd_row_stride":
            qkv = torch.empty(n, cols + 3, dtype=torch.bfloat16, device=gpu)[:, :cols]
        else:
            flat = torch.empty(n * (cols + 8) + 1, dtype=torch.bfloat16, device=gpu)
            qkv = flat[1:].view(n, cols + 8)[:, :cols]
        assert qkv.data_ptr() % 16 != 0 or qkv.stride(0) % 8 != 0
        qkv.copy_(case["qkv"])
        case["qkv"] = qkv
        case["pool"].copy_(pool0)
        case["out"].zero_()
        run(case)
        torch.cuda.synchronize()
    finally:
        ops.set_prefill_algorithm(saved)
    assert torch.equal(case["out"], ref_out)
    assert torch.equal(case["pool"], ref_pool)


@pytest.mark.parametrize("offset", [1, 2])
def test_norm_paths_agree_on_gate_alignment(gpu, offset):
    """The gated-RMSNorm pass after the chunked form reads `gate` with 16-byte pieces when
    its rows are 16-byte aligned, else two elements at a time (4-byte aligned rows) or one:
    gate rows shifted by `offset` elements (1: one element at a time, 2: pairs) give the
    aligned run's bits."""
    announce(test="prefill_norm_gate_alignment", offset=offset)
    case = prefill_case(gpu, [130, 64, 7, 200, 0, 65], seed=23)
    pool0 = case["pool"].clone()
    saved = ops.prefill_algorithm()
    ops.set_prefill_algorithm("chunked")
    try:
        run(case)
        torch.cuda.synchronize()
        ref_out, ref_pool = case["out"].clone(), case["pool"].clone()
        n, hv, d = case["gate"].shape
        storage = torch.empty(n, hv * d + offset, dtype=torch.bfloat16, device=gpu)
        gate = storage[:, offset:].unflatten(1, (hv, d))
        assert gate.data_ptr() % 16 != 0 and gate.stride(1) == d
        gate.copy_(case["gate"])
        case["gate"] = gate
        case["pool"].copy_(pool0)
        case["out"].zero_()
        run(case)
        torch.cuda.synchronize()
    finally:
        ops.set_prefill_algorithm(saved)
    assert torch.equal(case["out"], ref_out)
    assert torch.equal(case["pool"], ref_pool)


def test_rows_outside_every_sequence_are_left_alone(gpu, algorithm):
    """qkv rows that no sequence covers (all sequences empty here, or the tail after the
    last one): their outputs stay as they were; states are written back unchanged."""
    announce(test="prefill_uncovered_rows", algorithm=algorithm)
    for lengths, cu in (([3, 0], [0, 0, 0]), ([5, 4], [0, 5, 6])):
        case = prefill_case(gpu, lengths, seed=13)
        case["cu_seqlens"].copy_(torch.tensor(cu, dtype=torch.int32))
        case["out"].fill_(1.5)
        exp_out, exp_pool, pre = expected_prefill(*[case[k] for k in PREFILL], 1e-6,
                                                  return_pre=True)
        run(case)
        torch.cuda.synchronize()
        assert_bf16_outputs(case["out"], exp_out, pre, label=f"cu={cu}")
        assert torch.equal(case["out"][cu[-1]:].cpu(), exp_out[cu[-1]:])
        assert_states(case["pool"], exp_pool, label=f"cu={cu}")


@pytest.mark.parametrize("form", CHUNKED_FORMS)
@pytest.mark.parametrize("keys", ["identical", "alternating", "near_parallel"])
def test_chunked_with_adversarial_keys(gpu, keys, form):
    """Keys that make I + A of the WY form as far from the identity as it gets: every token
    of a sequence with the same key, keys of alternating sign, or keys within 1e-3 of each
    other; beta near 1 and decay near 1 (b = 6, a = -8).  The chunked form against the
    oracle's token-by-token recurrence, over 200 tokens (4 or 7 chunks)."""
    announce(test="prefill_chunked_adversarial", keys=keys, form=form)
    case = prefill_case(gpu, [200, 70], seed=21)
    saved = ops.prefill_algorithm()
    h, hv = 16, 32
    qkv = case["qkv"]
    k_cols = slice(h * 128, 2 * h * 128)
    gen = torch.Generator().manual_seed(22)
    base = torch.randn(1, h * 128, generator=gen)
    rows = qkv.shape[0]
    if keys == "identical":
        k = base.expand(rows, -1)
    elif keys == "alternating":
        k = base * torch.tensor([1.0, -1.0]).repeat(rows // 2 + 1)[:rows, None]
    else:
        k = base + 1e-3 * torch.randn(rows, h * 128, generator=gen)
    qkv[:, k_cols] = k.to(torch.bfloat16).to(gpu)
    case["b"].fill_(6.0)
    case["a"].fill_(-8.0)
    exp_out, exp_pool, pre = expected_prefill(*[case[k] for k in PREFILL], 1e-6, return_pre=True)
    try:
        ops.set_prefill_algorithm(form)
        run(case)
        torch.cuda.synchronize()
    finally:
        ops.set_prefill_algorithm(saved)
    assert_bf16_outputs(case["out"], exp_out, pre)
    assert_states(case["pool"], exp_pool)
