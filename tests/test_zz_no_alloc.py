"""ld_gdn_prefill_static (the prefill with its chunked workspace in the library's static
device scratch, allocating nothing) against ld_gdn_prefill with a caller workspace, through
the C ABI: the same kernels, so outputs and states must agree bit for bit.  Two calls in a
row, the second smaller (the scratch then holds the first call's contents), a shape whose
workspace exceeds the scratch (LD_PREFILL_AUTO then runs token-serial, like ld_gdn_prefill
without a workspace), and the refusal of a chunked prefill beyond the scratch."""

from __future__ import annotations

import pytest
import torch

from lightdelta_amd import _lib

pytestmark = pytest.mark.gpu

H, HV, DIM = 16, 32, 128


def announce(**what):
    print("case:", " ".join(f"{k}={v}" for k, v in what.items()), flush=True)


def prefill_case(lengths, seed, device):
    gen = torch.Generator(device=device).manual_seed(seed)
    total = sum(lengths)
    qkv_cols = (2 * H + HV) * DIM
    qkvz = torch.randn(total, qkv_cols + HV * DIM, generator=gen, device=device).bfloat16()
    ba = torch.randn(total, 2 * HV, generator=gen, device=device).bfloat16()
    n = len(lengths)
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32)
    return dict(
        qkv=qkvz[:, :qkv_cols], a=ba[:, HV:], b=ba[:, :HV],
        a_log=torch.rand(HV, generator=gen, device=device) * 2 - 1,
        dt_bias=torch.zeros(HV, device=device),
        slots=torch.arange(1, n + 1, dtype=torch.int32, device=device),
        has_initial=torch.ones(n, dtype=torch.bool, device=device),
        cu_seqlens=cu.to(device),
        pool=torch.empty(n + 1, HV, DIM, DIM, device=device).normal_(0.0, 0.02, generator=gen),
        gate=qkvz[:, qkv_cols:].view(total, HV, DIM),
        weight=1 + 0.1 * torch.randn(DIM, generator=gen, device=device),
        out=torch.zeros(total, HV, DIM, dtype=torch.bfloat16, device=device),
    )


def args_of(c, pool, out, algorithm, workspace=None):
    return _lib.PrefillArgs(
        c["qkv"].data_ptr(), c["qkv"].stride(0), c["a"].data_ptr(), c["a"].stride(0),
        c["b"].data_ptr(), c["b"].stride(0), c["a_log"].data_ptr(), c["dt_bias"].data_ptr(),
        _lib.DTYPE_F32, _lib.DTYPE_F32, c["slots"].data_ptr(), c["has_initial"].data_ptr(),
        c["cu_seqlens"].data_ptr(), pool.data_ptr(), pool.stride(0), c["gate"].data_ptr(),
        c["gate"].stride(0), c["weight"].data_ptr(), out.data_ptr(), c["qkv"].shape[0],
        c["slots"].numel(), H, HV, DIM**-0.5, 1e-6, algorithm,
        None if workspace is None else workspace.data_ptr(),
        0 if workspace is None else workspace.numel())


def run_both(c, algorithm, *, with_workspace=True):
    """(out, pool) of ld_gdn_prefill (caller workspace) and of ld_gdn_prefill_static."""
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    results = []
    for entry in ("ld_gdn_prefill", "ld_gdn_prefill_static"):
        pool, out = c["pool"].clone(), c["out"].clone()
        workspace = None
        if entry == "ld_gdn_prefill" and with_workspace:
            nbytes = lib.ld_gdn_prefill_workspace_bytes(c["qkv"].shape[0], c["slots"].numel(), HV)
            workspace = torch.empty(nbytes, dtype=torch.uint8, device=pool.device)
        _lib.check(getattr(lib, entry)(args_of(c, pool, out, algorithm, workspace), stream))
        torch.cuda.synchronize()
        results.append((out.cpu(), pool.cpu()))
    return results


def assert_same(results, label):
    (out_ref, pool_ref), (out_static, pool_static) = results
    assert torch.equal(out_ref.view(torch.int16), out_static.view(torch.int16)), f"{label}: out"
    assert torch.equal(pool_ref, pool_static), f"{label}: state"
    assert out_ref.abs().sum() > 0, f"{label}: nothing written"


def test_static_scratch_matches_caller_workspace_twice(gpu):
    """Two calls in a row, the second with a smaller input, chunked form forced; then AUTO
    and the 32-token form."""
    first = prefill_case([300, 337], seed=1, device=gpu)
    need = _lib.load().ld_gdn_prefill_workspace_bytes(637, 2, HV)
    assert need <= _lib.PREFILL_STATIC_SCRATCH_BYTES
    announce(test="no_alloc", call=1, tokens=637, workspace=need)
    assert_same(run_both(first, _lib.PREFILL_CHUNKED), "first call")
    second = prefill_case([130], seed=2, device=gpu)
    announce(test="no_alloc", call=2, tokens=130)
    assert_same(run_both(second, _lib.PREFILL_CHUNKED), "second call")
    announce(test="no_alloc", call=3, tokens=130, algorithm="auto")
    assert_same(run_both(second, _lib.PREFILL_AUTO), "auto")
    announce(test="no_alloc", call=4, tokens=637, algorithm="chunked_32")
    assert_same(run_both(first, _lib.PREFILL_CHUNKED_32), "32-token chunks")


def test_static_beyond_scratch_runs_token_serial_or_refuses(gpu):
    """A workspace beyond the scratch: AUTO runs token-serial (as ld_gdn_prefill without a
    workspace does), CHUNKED is refused and writes nothing."""
    case = prefill_case([1024] * 4, seed=3, device=gpu)
    lib = _lib.load()
    assert lib.ld_gdn_prefill_workspace_bytes(4096, 4, HV) > _lib.PREFILL_STATIC_SCRATCH_BYTES
    announce(test="no_alloc_beyond", tokens=4096)
    assert_same(run_both(case, _lib.PREFILL_AUTO, with_workspace=False), "beyond, auto")
    out = case["out"].clone()
    rc = lib.ld_gdn_prefill_static(args_of(case, case["pool"], out, _lib.PREFILL_CHUNKED),
                                   torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 1 and b"static scratch" in lib.ld_last_error()
    assert out.abs().sum() == 0
