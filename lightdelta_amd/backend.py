"""The post-convolution compute / state-access boundary (drop-in for the reference's
`lightdelta.backend.GDNBackend`, python/lightdelta/backend.py:12-91).

    backend = GDNBackend(config)
    backend(qkv, a, b, a_log, dt_bias, slots, cu, accepted, pool, gate, weight, out, eps)

* state_io = "indexed": one `torch.ops.lightdelta.decode` launch straight on the pool.
* state_io = "packed": the source state of every request is gathered into a cached scratch
  buffer (row 0 reserved, request r's T rows at 1 + r*T), the step runs on the scratch, and
  the per-token states are written back to their slots.  With compute = "cuda_fused" the
  bookkeeping (sources, validity, scratch rows, destinations: one packed_plan launch), the
  gather, the step and the write-back are the gfx950 HIP kernels; with "torch_reference"
  (an eager ablation) they are plain torch index ops plus the unfused Torch GDN.

Semantics shared by both paths (reference backend.py:39-47, 87-91):
  source  = slots[r, clamp(accepted[r], 1, T) - 1]
  valid   = 1 <= accepted[r] <= T and source > 0        (else: zero output, no write)
  live    = t < cu[r+1] - cu[r]
  the state after token t goes to slots[r, t] when live and valid and slots[r, t] > 0;
  slot 0 (and any slot <= 0) is never written.
Nothing here reads device memory on the host, so the fused paths are graph-capturable once
the scratch for a (device, batch, width) key exists (created on the first, eager, call).
"""

from __future__ import annotations

from collections import Counter

import torch

from . import ops  # noqa: F401  -- registers torch.ops.lightdelta
from .config import BackendConfig
from .torch_gdn import GDNInputs, post_conv_gdn

HEAD_DIM = 128


class GDNBackend:
    def __init__(self, config: BackendConfig):
        config.validate()
        self.config = config
        self.calls = Counter()
        self._packed = {}

    def __call__(
        self, qkv, a, b, a_log, dt_bias, slots, cu, accepted, pool, gate, weight, out, eps=1e-6
    ):
        batch, width = slots.shape
        self.calls["decode" if width == 1 else "verify"] += 1
        if self.config.state_io == "indexed":
            torch.ops.lightdelta.decode(
                qkv, a, b, a_log, dt_bias, slots, cu, accepted, pool, gate, weight, out, eps
            )
            return

        scratch, ones, offsets, plan = self._scratch(pool, batch, width)
        initial = scratch[1:].view(batch, width, *pool.shape[1:])[:, 0]

        if self.config.compute == "cuda_fused":
            # source, valid, indices and destinations of the semantics above, in one launch
            source, valid, indices, destinations = plan
            torch.ops.lightdelta.packed_plan(slots, cu, accepted, source, valid, indices,
                                             destinations)
            torch.ops.lightdelta.gather_state(pool, source, valid, initial)
            torch.ops.lightdelta.decode(
                qkv, a, b, a_log, dt_bias, indices, cu, ones, scratch, gate, weight, out, eps
            )
            torch.ops.lightdelta.scatter_state(scratch[1:], destinations, pool)
            return

        source = slots.gather(1, (accepted.clamp(1, width) - 1)[:, None].long()).flatten()
        valid = (accepted > 0) & (accepted <= width) & (source > 0)
        lengths = cu[1:] - cu[:-1]
        live = offsets < lengths[:, None]
        destinations = torch.where(live & valid[:, None] & (slots > 0), slots, 0).flatten()

        # compute == "torch_reference": eager torch ops end to end.
        torch.index_select(pool, 0, source.clamp_min(0).long(), out=initial)
        initial.masked_fill_(~valid[:, None, None, None], 0)
        states = self._torch_step(
            qkv, a, b, a_log, dt_bias, cu, offsets, live, valid, lengths, initial, gate, weight,
            out, eps, batch, width, pool,
        )
        keep = destinations[:, None, None, None] > 0
        pool.index_copy_(0, destinations.long(), torch.where(keep, states, pool[0]))

    def _scratch(self, pool, batch, width):
        key = (pool.device, batch, width)
        cached = self._packed.get(key)
        if cached is None:
            device = pool.device
            cached = (
                pool.new_empty((1 + batch * width, *pool.shape[1:])),
                torch.ones(batch, device=device, dtype=torch.int32),
                torch.arange(width, device=device, dtype=torch.int32)[None, :],
                # the fused path's bookkeeping outputs (packed_plan): source, valid,
                # indices, destinations
                (torch.empty(batch, device=device, dtype=torch.int32),
                 torch.empty(batch, device=device, dtype=torch.bool),
                 torch.empty(batch, width, device=device, dtype=torch.int32),
                 torch.empty(batch * width, device=device, dtype=torch.int32)),
            )
            self._packed[key] = cached
        return cached

    @staticmethod
    def _torch_step(
        qkv, a, b, a_log, dt_bias, cu, offsets, live, valid, lengths, initial, gate, weight,
        out, eps, batch, width, pool,
    ):
        value_heads = pool.shape[1]
        key_heads = (qkv.shape[1] // HEAD_DIM - value_heads) // 2
        token_ids = cu[:-1, None] + offsets
        if width == 1:
            rows = [x.unsqueeze(1) for x in (qkv, a, b, gate)]
        else:
            ids = token_ids.clamp(0, qkv.shape[0] - 1).long()
            rows = [x[ids] for x in (qkv, a, b, gate)]
        dense, ad, bd, gd = rows
        q, k, v = dense.split(
            (key_heads * HEAD_DIM, key_heads * HEAD_DIM, value_heads * HEAD_DIM), dim=-1
        )
        result = post_conv_gdn(
            GDNInputs(
                q.reshape(batch, width, key_heads, HEAD_DIM),
                k.reshape(batch, width, key_heads, HEAD_DIM),
                v.reshape(batch, width, value_heads, HEAD_DIM),
                ad,
                bd,
                a_log,
                dt_bias,
                gd,
                weight,
            ),
            initial,
            torch.where(valid, lengths, 0),
            save_checkpoints=width > 1,
            norm_eps=eps,
        )
        if width == 1:
            out.copy_(result.output[:, 0])
            return result.final_state
        out.index_copy_(0, token_ids[live].long(), result.output[live])
        return result.checkpoints[:, 1:].reshape(batch * width, *pool.shape[1:])
