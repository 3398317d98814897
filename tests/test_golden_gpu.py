"""The HIP decode against the reference's own outputs: the golden vectors that
tests/golden/make_golden.py wrote with the reference's post_conv_gdn
(python/lightdelta/reference/gdn.py:70-128) at the workload's first configuration (B=1,
4 qk / 8 v heads, dk = dv = 128).  The kernel runs those shapes natively, so its outputs and
states are compared with the stored ones directly, not only through the oracle:

  cfg1_step  one token from the stored initial state;
  cfg1_64    64 consecutive tokens, the state carried on the GPU from step to step (the
             reference wrote them as one 64-token call, which equals 64 single steps).

Outputs: within rtol = atol = 2e-3 of the stored bf16 outputs, except elements whose
rounding sits on a bf16 midpoint (flagged from the oracle's pre-rounding values on the same
inputs; the oracle reproduces these vectors bit for bit, test_oracle.py); states after 64
steps within rtol = atol = 2e-3, after one step within the reference's own 3e-4 / 3e-6
(tests/test_gdn.py:74).  Both state cache policies run (they use different kernels for one
token), through the op and through GDNBackend in indexed and packed mode."""

from __future__ import annotations

import pytest
import torch

from lightdelta_amd import ops
from lightdelta_amd.backend import GDNBackend
from lightdelta_amd.config import BackendConfig
from oracle import gdn
from tests.parity import assert_bf16_outputs, assert_states

pytestmark = pytest.mark.gpu

STEP_STATE = dict(rtol=3e-4, atol=3e-6)


def announce(**what):
    print("case:", " ".join(f"{k}={v}" for k, v in what.items()), flush=True)


@pytest.fixture(params=["keep", "stream"])
def policy(request):
    saved = ops.state_cache_policy()
    ops.set_state_cache_policy(request.param)
    yield request.param
    ops.set_state_cache_policy(saved)


class Layer:
    """Device buffers of one B=1 decode layer in the production layout (qkv and gate column
    slices of one [1, qkv + gate] buffer, a and b slices of one [1, 2*HV] buffer), with the
    state in slot 1 of a 3-slot pool whose slots 0 and 2 hold sentinels."""

    def __init__(self, d, device):
        self.h = d["q"].shape[2]
        self.hv = d["v"].shape[2]
        qkv_cols = (2 * self.h + self.hv) * 128
        self.qkv_cols = qkv_cols
        self.qkvz = torch.zeros(1, qkv_cols + self.hv * 128, dtype=torch.bfloat16, device=device)
        self.ba = torch.zeros(1, 2 * self.hv, dtype=torch.bfloat16, device=device)
        self.pool = torch.randn(3, self.hv, 128, 128, generator=torch.Generator().manual_seed(3)
                                ).to(device)
        self.sentinel = self.pool[[0, 2]].clone()
        self.pool[1] = d["state"][0].to(device)
        self.a_log = d["a_log"].to(device)
        self.dt_bias = d["dt_bias"].to(device)
        self.weight = d["norm_weight"].to(device)
        self.slots = torch.tensor([[1]], dtype=torch.int32, device=device)
        self.cu = torch.tensor([0, 1], dtype=torch.int32, device=device)
        self.accepted = torch.ones(1, dtype=torch.int32, device=device)
        self.out = torch.zeros(1, self.hv, 128, dtype=torch.bfloat16, device=device)

    def load_token(self, d, t):
        row = torch.cat([d["q"][0, t].reshape(-1), d["k"][0, t].reshape(-1),
                         d["v"][0, t].reshape(-1), d["gate"][0, t].reshape(-1)])
        self.qkvz.copy_(row[None].to(self.qkvz.device))
        self.ba.copy_(torch.cat([d["b"][0, t], d["a"][0, t]])[None].to(self.ba.device))

    def args(self):
        return (self.qkvz[:, : self.qkv_cols], self.ba[:, self.hv:], self.ba[:, : self.hv],
                self.a_log, self.dt_bias, self.slots, self.cu, self.accepted, self.pool,
                self.qkvz[:, self.qkv_cols:].view(1, self.hv, 128), self.weight, self.out)


def oracle_pre(d, t, state):
    """The oracle's step t from `state` (fp32 [1, HV, 128, 128]): its output, new state and
    pre-rounding values, which flag the rounding-sensitive elements.  (The oracle equals the
    stored vectors bit for bit on the CPU that wrote them, test_oracle.py; another CPU's
    summation order may move a few of them by one ulp, so that is not asserted here.)"""
    step = [d[f][:, t:t + 1] for f in ("q", "k", "v", "a", "b")]
    out, new_state, _, (raw, y) = gdn.run(*step, d["a_log"], d["dt_bias"], d["gate"][:, t:t + 1],
                                          d["norm_weight"], state, d["lengths"], return_pre=True)
    return out[0, 0], new_state, (raw[0, 0], y[0, 0])


def run_step(layer, mode):
    if mode == "op":
        torch.ops.lightdelta.decode(*layer.args(), 1e-6)
    else:
        GDNBackend(BackendConfig(compute="cuda_fused", state_io=mode))(*layer.args(), 1e-6)


@pytest.mark.parametrize("mode", ["op", "indexed", "packed"])
def test_reference_single_step(gpu, golden, policy, mode):
    announce(test="golden_cfg1_step", policy=policy, mode=mode)
    d = golden("cfg1_step")
    layer = Layer(d, gpu)
    layer.load_token(d, 0)
    run_step(layer, mode)
    torch.cuda.synchronize()
    _, _, pre = oracle_pre(d, 0, d["state"])
    assert_bf16_outputs(layer.out[0], d["output"][0, 0], pre, label="cfg1_step out")
    assert_states(layer.pool[1][None], d["final_state"], label="cfg1_step state", **STEP_STATE)
    assert torch.equal(layer.pool[[0, 2]].cpu(), layer.sentinel.cpu()), "untouched slots changed"


@pytest.mark.parametrize("mode", ["op", "packed"])
def test_reference_64_steps(gpu, golden, policy, mode):
    announce(test="golden_cfg1_64", policy=policy, mode=mode)
    d = golden("cfg1_64")
    layer = Layer(d, gpu)
    state = d["state"]
    flips = 0
    for t in range(64):
        layer.load_token(d, t)
        run_step(layer, mode)
        _, state, pre = oracle_pre(d, t, state)
        flips += assert_bf16_outputs(layer.out[0], d["output"][0, t], pre,
                                     label=f"cfg1_64 step {t}")["flips"]
    torch.cuda.synchronize()
    assert_states(layer.pool[1][None], d["final_state"], label="cfg1_64 state after 64 steps")
    drift = ((layer.pool[1].cpu() - d["final_state"][0]).abs().max()
             / d["final_state"].abs().max()).item()
    assert torch.equal(layer.pool[[0, 2]].cpu(), layer.sentinel.cpu()), "untouched slots changed"
    print(f"golden 64 steps ({policy}, {mode}): {flips} rounding flips of {64 * 8 * 128}, "
          f"max state difference {drift:.2e} of max |state|")
