"""Bit-exact parity of the gfx950 state-pool copies with the numpy oracle (small pools),
the reference's own gather/scatter test (tests/test_gdn.py:125-143), and size-independent
properties at the workload size (1024-slot fp32 pool, bf16 conv pool, 128 pairs)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import state_io as oracle

pytestmark = pytest.mark.gpu


def announce(**what):
    print("case:", " ".join(f"{k}={v}" for k, v in what.items()), flush=True)


@pytest.mark.parametrize("index_stride", [1, 4])
def test_prefill_state_initialization_and_reuse(gpu, index_stride):
    """Reference tests/test_gdn.py:125-143: strided slots, valid mask, padding slot 0."""
    announce(test="prefill_init_reuse", stride=index_stride)
    gen = torch.Generator().manual_seed(42)
    pool = (torch.randn(6, 48, 128, 128, generator=gen) * 0.1).to(gpu)
    before = pool.clone()
    slots = torch.full((3, index_stride), -1, device=gpu, dtype=torch.int32)[:, 0]
    slots.copy_(torch.tensor([2, 1, 0], device=gpu, dtype=torch.int32))
    valid = torch.tensor([True, False, False], device=gpu)
    packed = torch.empty(3, *pool.shape[1:], device=gpu)
    torch.ops.lightdelta.gather_state(pool, slots, valid, packed)
    torch.cuda.synchronize()
    assert torch.equal(packed[0], pool[2])
    assert packed[1:].count_nonzero() == 0
    packed.add_(1)
    torch.ops.lightdelta.scatter_state(packed, slots, pool)
    torch.cuda.synchronize()
    assert torch.equal(pool[0], before[0])
    assert torch.equal(pool[1], torch.ones_like(pool[1]))
    assert torch.equal(pool[2], before[2] + 1)


def row_bytes(t: torch.Tensor) -> np.ndarray:
    """Bit patterns of a pool-shaped tensor as a [rows, bytes] uint8 array."""
    return t.detach().cpu().contiguous().view(torch.uint8).reshape(t.shape[0], -1).numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.int32])
def test_gather_scatter_copy_match_numpy(gpu, dtype):
    announce(test="gather_scatter_copy", dtype=dtype)
    gen = torch.Generator().manual_seed(0)
    slots_n, shape = 40, (3, 64, 8)
    raw = torch.randint(-2**15, 2**15, (slots_n, *shape, 4 // 2), generator=gen, dtype=torch.int16)
    # random bit patterns reinterpreted as `dtype` (bit-exact copies do not care about values)
    pool = raw.view(torch.uint8).view(dtype).reshape(slots_n, *shape, -1)[..., 0].contiguous().to(gpu)
    host = row_bytes(pool)
    slots = torch.tensor([5, 0, -1, 17, 39, 5, 2], dtype=torch.int32)
    valid = torch.tensor([True, True, True, False, True, True, True])
    out = torch.empty(len(slots), *shape, dtype=dtype, device=gpu)
    torch.ops.lightdelta.gather_slots(pool, slots.to(gpu), valid.to(gpu), out)
    assert np.array_equal(row_bytes(out), oracle.gather(host, slots.numpy(), valid.numpy()))

    packed = torch.flip(out, [0]).contiguous()
    dst = torch.tensor([3, 0, 9, -1, 12, 30, 31], dtype=torch.int32)
    torch.ops.lightdelta.scatter_slots(packed, dst.to(gpu), pool)
    expected = oracle.scatter(row_bytes(packed), dst.numpy(), host)
    assert np.array_equal(row_bytes(pool), expected)

    src = torch.tensor([1, -1, 7, 8, 0, 20], dtype=torch.int32)
    dst = torch.tensor([2, 3, -1, 9, 10, 21], dtype=torch.int32)
    torch.ops.lightdelta.copy_state(pool, src.to(gpu), dst.to(gpu))
    assert np.array_equal(row_bytes(pool), oracle.copy(expected, src.numpy(), dst.numpy()))
    copied = oracle.copy(expected, src.numpy(), dst.numpy())

    reset = torch.tensor([4, -1, 0, 38, 11], dtype=torch.int32)
    torch.ops.lightdelta.zero_slots(pool, reset.to(gpu))
    assert np.array_equal(row_bytes(pool), oracle.zero(copied, reset.numpy()))


def test_copy_state_overlapping_pairs(gpu):
    """Pair sets with a chain, a cycle, two writes of one slot, a self pair, padding and
    independent pairs, on a pool of 2 MiB slots (every chunk of a row must agree): bit-exact
    against the oracle, which rejects every overlapping pair."""
    announce(test="copy_state_overlapping_pairs")
    gen = torch.Generator().manual_seed(5)
    pool = torch.randn(24, 32, 128, 128, generator=gen).to(gpu)
    host = row_bytes(pool)
    src = torch.tensor([1, 2, 4, 5, 6, 8, 10, 11, -1, 13, 14, 16, 20], dtype=torch.int32)
    dst = torch.tensor([2, 3, 5, 6, 4, 9, 10, -1, 8, 12, 12, 17, 21], dtype=torch.int32)
    torch.ops.lightdelta.copy_state(pool, src.to(gpu), dst.to(gpu))
    torch.cuda.synchronize()
    expected = oracle.copy(host, src.numpy(), dst.numpy())
    assert np.array_equal(row_bytes(pool), expected)
    assert not np.array_equal(expected[[9, 17, 21]], host[[9, 17, 21]])  # some pairs applied
    assert np.array_equal(expected[[2, 3, 4, 5, 6, 12]], host[[2, 3, 4, 5, 6, 12]])


def test_copy_state_checked_reports_rejected_pairs(gpu):
    """copy_state_checked on pair sets with a chain (1->2, 2->3), a swap (4<->5), a shared
    destination (7->9, 8->9), a self pair, padding and independent pairs, on 2 MiB slots:
    the pool is bit-exact against the oracle (as copy_state), and `rejected` holds 1 exactly
    for the pairs the oracle rejects and 0 for the others, padding included.  The status
    array starts full of garbage (every entry is written), and a HIP-graph replay with new
    pairs reports them the same way."""
    announce(test="copy_state_checked")
    gen = torch.Generator().manual_seed(6)
    pool = torch.randn(24, 32, 128, 128, generator=gen).to(gpu)
    src = torch.tensor([1, 2, 4, 5, 7, 8, 10, -1, 13, 15, 0, 18], dtype=torch.int32)
    dst = torch.tensor([2, 3, 5, 4, 9, 9, 10, 11, 14, -1, 16, 19], dtype=torch.int32)
    rejected = torch.full((len(src),), 7, dtype=torch.int32, device=gpu)
    host = row_bytes(pool)
    src_d, dst_d = src.to(gpu), dst.to(gpu)
    torch.ops.lightdelta.copy_state_checked(pool, src_d, dst_d, rejected)
    torch.cuda.synchronize()
    expected_rejected = oracle.copy_rejected(src.numpy(), dst.numpy())
    assert list(expected_rejected) == [True, True, True, True, True, True, False, False, False,
                                       False, False, False]
    assert np.array_equal(rejected.cpu().numpy(), expected_rejected.astype(np.int32))
    assert int(rejected.sum()) == 6
    assert np.array_equal(row_bytes(pool), oracle.copy(host, src.numpy(), dst.numpy()))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        torch.ops.lightdelta.copy_state_checked(pool, src_d, dst_d, rejected)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        torch.ops.lightdelta.copy_state_checked(pool, src_d, dst_d, rejected)
    for replay, (s_new, d_new) in enumerate((
            ([3, 6, 20, 21, -1, 12, 1, 2, 9, 22, 23, 17], [6, 20, 21, 3, 4, 13, 2, 1, 8, 23, 22, 12]),
            ([1, 3, 5, 7, 9, 11, 13, 15, 17, 19, 21, 23], [2, 4, 6, 8, 10, 12, 14, 16, 18, 20, 22, 0]))):
        s_t = torch.tensor(s_new, dtype=torch.int32)
        d_t = torch.tensor(d_new, dtype=torch.int32)
        src_d.copy_(s_t)
        dst_d.copy_(d_t)
        rejected.fill_(-3)
        host = row_bytes(pool)
        graph.replay()
        torch.cuda.synchronize()
        exp = oracle.copy_rejected(s_t.numpy(), d_t.numpy()).astype(np.int32)
        assert np.array_equal(rejected.cpu().numpy(), exp), f"replay {replay}"
        assert np.array_equal(row_bytes(pool), oracle.copy(host, s_t.numpy(), d_t.numpy()))
        assert int(exp.sum()) == (10, 0)[replay]  # a 4-cycle, two swaps, a chain 17->12->13


def test_gather_into_strided_rows(gpu):
    """The packed backend gathers into scratch[1:].view(B, W, ...)[:, 0] (row stride W)."""
    announce(test="gather_strided_rows")
    pool = torch.randn(9, 4, 128, 128, device=gpu)
    scratch = torch.full((1 + 3 * 2, 4, 128, 128), 7.0, device=gpu)
    rows = scratch[1:].view(3, 2, 4, 128, 128)[:, 0]
    slots = torch.tensor([8, 0, 3], device=gpu, dtype=torch.int32)
    valid = torch.tensor([True, True, False], device=gpu)
    torch.ops.lightdelta.gather_state(pool, slots, valid, rows)
    torch.cuda.synchronize()
    assert torch.equal(rows[0], pool[8])
    assert rows[1:].count_nonzero() == 0
    assert torch.equal(scratch[2], torch.full_like(scratch[2], 7.0))  # odd rows untouched


def test_workload_pool_copies(gpu):
    """1024-slot fp32 pool (32 x 128 x 128 per slot, 2 GiB) and bf16 conv pool (4 x 8192 per
    slot): gather 128 slots, scatter them back to other slots, slot-to-slot copy of 128
    random pairs including padding -1, reset of 128 slots -- each bit-exact against the
    pool itself."""
    announce(test="workload_pool_copies")
    gen = torch.Generator(device="cpu").manual_seed(0)
    for shape, dtype in (((32, 128, 128), torch.float32), ((4, 8192), torch.bfloat16)):
        pool = torch.randn(1024, *shape, device=gpu, dtype=torch.float32).to(dtype)
        before = pool.clone()
        perm = torch.randperm(1023, generator=gen) + 1
        src = perm[:128].to(torch.int32)
        dst = perm[128:256].to(torch.int32)
        src[::17] = -1
        dst[5::23] = -1
        packed = torch.empty(128, *shape, device=gpu, dtype=dtype)
        valid = torch.ones(128, dtype=torch.bool, device=gpu)
        torch.ops.lightdelta.gather_slots(pool, src.to(gpu), valid, packed)
        live = (src > 0).to(gpu)
        assert torch.equal(packed[live], pool[src.clamp_min(0).long().to(gpu)][live])
        assert packed[~live].count_nonzero() == 0
        torch.ops.lightdelta.scatter_slots(packed, dst.to(gpu), pool)
        ok = (dst > 0).to(gpu)
        assert torch.equal(pool[dst.clamp_min(0).long().to(gpu)][ok], packed[ok])
        pool.copy_(before)
        torch.ops.lightdelta.copy_state(pool, src.to(gpu), dst.to(gpu))
        torch.cuda.synchronize()
        moved = ((src > 0) & (dst > 0)).to(gpu)
        d, s = dst.long().to(gpu)[moved], src.long().to(gpu)[moved]
        assert torch.equal(pool[d], before[s])
        untouched = torch.ones(1024, dtype=torch.bool, device=gpu)
        untouched[d] = False
        assert torch.equal(pool[untouched], before[untouched])
        # reset 128 slots for reuse (with padding ids), the rest untouched
        reset = (torch.randperm(1023, generator=gen)[:128] + 1).to(torch.int32)
        reset[3::29] = -1
        after_copy = pool.clone()
        torch.ops.lightdelta.zero_slots(pool, reset.to(gpu))
        torch.cuda.synchronize()
        cleared = torch.zeros(1024, dtype=torch.bool, device=gpu)
        cleared[reset[reset > 0].long().to(gpu)] = True
        assert pool[cleared].count_nonzero() == 0
        assert torch.equal(pool[~cleared], after_copy[~cleared])
        del pool, before, packed, after_copy
        torch.cuda.empty_cache()
