"""Slot-indexed decode / MTP-verify semantics on top of oracle.gdn -- test infrastructure.

`expected_decode` restates what one `lightdelta::decode` call does to `out` and the state
pool (reference csrc/gdn_decode.cu:142-168 and 303-316, backend.py:39-47):
  * request r covers tokens cu[r] .. cu[r+1]-1 (n tokens); n <= 0: nothing is written;
  * source slot = indices[r, accepted[r]-1] if 1 <= accepted[r] <= W, else 0;
  * source <= 0: the request's outputs are zero and the pool is untouched;
  * otherwise the request runs n tokens from pool[source]; the state after token t is
    written to indices[r, t] when that slot is > 0.
  * n > W: treated as invalid (zero outputs, no writes).  The reference kernel would read
    the next request's indices there (csrc/gdn_decode.cu:303-304); this build bounds it.
All sources are read before any write, as in a launch whose requests touch disjoint slots.

`expected_prefill` restates the layer's prefill (reference
python/lightdelta/integration/vllm_layer.py:93-135 with prefill_io = "fused_copy"): per
sequence n (rows cu_seqlens[n] .. cu_seqlens[n+1]-1) the initial state is pool[slots[n]]
when slots[n] > 0 and has_initial[n], else zeros (gather_state's zero fill); the sequence
runs post_conv_gdn over its tokens; the final state goes to pool[slots[n]] when
slots[n] > 0 (scatter_state skips padding).

`packed_reference_step` is the reference's Torch path (backend.py:30-91 with
compute="torch_reference"): gather with index_select, the unfused GDN, write back with
index_copy_.  It mutates `pool` and `out` in place; bench.py times it as the CPU baseline.
"""

from __future__ import annotations

import torch

from . import conv as conv_oracle
from . import gdn

HEAD_DIM = 128


def geometry(qkv: torch.Tensor, pool: torch.Tensor) -> tuple[int, int]:
    hv = pool.shape[1]
    h = (qkv.shape[1] // HEAD_DIM - hv) // 2
    return h, hv


def split_tokens(qkv, a, b, gate, rows, h, hv):
    """Per-token q, k, v, a, b, gate of `rows` (a slice or index tensor) as [1, n, ...]."""
    x = qkv[rows]
    n = x.shape[0]
    q = x[:, : h * HEAD_DIM].reshape(1, n, h, HEAD_DIM)
    k = x[:, h * HEAD_DIM: 2 * h * HEAD_DIM].reshape(1, n, h, HEAD_DIM)
    v = x[:, 2 * h * HEAD_DIM: (2 * h + hv) * HEAD_DIM].reshape(1, n, hv, HEAD_DIM)
    return q, k, v, a[rows][None], b[rows][None], gate[rows][None]


def expected_decode(qkv, a, b, a_log, dt_bias, indices, cu, accepted, pool, gate, weight, out,
                    eps, *, return_pre=False):
    """Expected (out, pool) after one decode call, as new CPU tensors.  With return_pre,
    also (raw_pre, y_pre) [N, HV, 128] fp32 (zero where the oracle wrote no value)."""
    qkv, a, b, a_log, dt_bias, gate, weight = (
        t.cpu() for t in (qkv, a, b, a_log, dt_bias, gate, weight))
    indices, cu, accepted = indices.cpu().long(), cu.cpu().long(), accepted.cpu().long()
    new_out = out.cpu().clone()
    new_pool = pool.cpu().clone()
    source_pool = pool.cpu()
    h, hv = geometry(qkv, source_pool)
    requests, width = indices.shape
    raw_pre = torch.zeros(new_out.shape, dtype=torch.float32)
    y_pre = torch.zeros(new_out.shape, dtype=torch.float32)
    writes = []
    for r in range(requests):
        bos, eos = int(cu[r]), int(cu[r + 1])
        n = eos - bos
        if n <= 0:
            continue
        acc = int(accepted[r])
        source = int(indices[r, acc - 1]) if 1 <= acc <= width else 0
        if source <= 0 or n > width:
            new_out[bos:eos] = 0
            continue
        q, k, v, ar, br, gr = split_tokens(qkv, a, b, gate, slice(bos, eos), h, hv)
        o, _, ckpt, (raw, y) = gdn.run(
            q, k, v, ar, br, a_log, dt_bias, gr, weight, source_pool[source][None],
            torch.tensor([n]), save_checkpoints=True, norm_eps=eps, return_pre=True)
        new_out[bos:eos] = o[0]
        raw_pre[bos:eos] = raw[0]
        y_pre[bos:eos] = y[0]
        for t in range(n):
            dest = int(indices[r, t])
            if dest > 0:
                writes.append((dest, ckpt[0, t + 1]))
    for dest, state in writes:
        new_pool[dest] = state
    if return_pre:
        return new_out, new_pool, (raw_pre, y_pre)
    return new_out, new_pool


def expected_prefill(qkv, a, b, a_log, dt_bias, slots, has_initial, cu_seqlens, pool, gate,
                     weight, out, eps, *, return_pre=False):
    """Expected (out, pool) after one prefill call, as new CPU tensors; with return_pre also
    (raw_pre, y_pre) [T, HV, 128] fp32 (zero on rows no sequence covers)."""
    qkv, a, b, a_log, dt_bias, gate, weight = (
        t.cpu() for t in (qkv, a, b, a_log, dt_bias, gate, weight))
    slots, cu = slots.cpu().long(), cu_seqlens.cpu().long()
    has_initial = has_initial.cpu()
    new_out = out.cpu().clone()
    new_pool = pool.cpu().clone()
    source_pool = pool.cpu()
    h, hv = geometry(qkv, source_pool)
    raw_pre = torch.zeros(new_out.shape, dtype=torch.float32)
    y_pre = torch.zeros(new_out.shape, dtype=torch.float32)
    writes = []
    for n in range(slots.numel()):
        bos, eos = int(cu[n]), int(cu[n + 1])
        slot = int(slots[n])
        if slot > 0 and bool(has_initial[n]):
            initial = source_pool[slot].clone()
        else:
            initial = torch.zeros(source_pool.shape[1:], dtype=source_pool.dtype)
        final = initial
        if eos > bos:
            q, k, v, ar, br, gr = split_tokens(qkv, a, b, gate, slice(bos, eos), h, hv)
            o, final, _, (raw, y) = gdn.run(
                q, k, v, ar, br, a_log, dt_bias, gr, weight, initial[None],
                torch.tensor([eos - bos]), norm_eps=eps, return_pre=True)
            final = final[0]
            new_out[bos:eos] = o[0]
            raw_pre[bos:eos] = raw[0]
            y_pre[bos:eos] = y[0]
        if slot > 0:
            writes.append((slot, final))
    for slot, state in writes:
        new_pool[slot] = state
    if return_pre:
        return new_out, new_pool, (raw_pre, y_pre)
    return new_out, new_pool


def packed_reference_step(qkv, a, b, a_log, dt_bias, slots, cu, accepted, pool, gate, weight,
                          out, eps, scratch=None):
    """The reference's packed Torch path, in place on `pool` and `out` (backend.py:30-91).
    `scratch` ([1 + B*W, *pool.shape[1:]]) may be passed in to keep allocation out of a
    timed loop."""
    batch, width = slots.shape
    h, hv = geometry(qkv, pool)
    if scratch is None:
        scratch = pool.new_empty((1 + batch * width, *pool.shape[1:]))
    source = slots.gather(1, (accepted.clamp(1, width) - 1)[:, None].long()).flatten()
    valid = (accepted > 0) & (accepted <= width) & (source > 0)
    initial = scratch[1:].view(batch, width, *pool.shape[1:])[:, 0]
    torch.index_select(pool, 0, source.clamp_min(0).long(), out=initial)
    initial.masked_fill_(~valid[:, None, None, None], 0)
    lengths = cu[1:] - cu[:-1]
    offsets = torch.arange(width)[None, :]
    live = offsets < lengths[:, None]
    token_ids = cu[:-1, None] + offsets
    if width == 1:
        dense, ad, bd, gd = (x.unsqueeze(1) for x in (qkv, a, b, gate))
    else:
        ids = token_ids.clamp(0, qkv.shape[0] - 1).long()
        dense, ad, bd, gd = (x[ids] for x in (qkv, a, b, gate))
    q = dense[..., : h * HEAD_DIM].reshape(batch, width, h, HEAD_DIM)
    k = dense[..., h * HEAD_DIM: 2 * h * HEAD_DIM].reshape(batch, width, h, HEAD_DIM)
    v = dense[..., 2 * h * HEAD_DIM:].reshape(batch, width, hv, HEAD_DIM)
    output, final, ckpt = gdn.run(
        q, k, v, ad, bd, a_log, dt_bias, gd, weight, initial, torch.where(valid, lengths, 0),
        save_checkpoints=width > 1, norm_eps=eps)
    if width == 1:
        out.copy_(output[:, 0])
        states = final
    else:
        out.index_copy_(0, token_ids[live].long(), output[live])
        states = ckpt[:, 1:].reshape(batch * width, *pool.shape[1:])
    destinations = torch.where(live & valid[:, None] & (slots > 0), slots, 0).flatten()
    keep = destinations[:, None, None, None] > 0
    pool.index_copy_(0, destinations.long(), torch.where(keep, states, pool[0]))


def expected_decode_conv(mixed_qkv, conv_state, conv_weight, conv_bias, a, b, a_log, dt_bias,
                         indices, cu, accepted, pool, gate, weight, out, eps, *, return_pre=False):
    """Expected (out, pool, conv_state) after one conv-fused decode / verify call: the conv
    update (oracle/conv.py, conv_update_tokens) of every request's tokens on conv slot
    indices[r, 0] from column offset accepted[r] - 1, then expected_decode on the post-conv
    activations.  A request is processed only if the GDN step accepts it and its conv
    columns lie in the state (conv slot > 0, offset + 2 <= S - 1, and offset <= n - 1 unless
    n >= S); otherwise its outputs are zero and neither pool changes.
    Returns (out, pool[, pre], conv_state, post), post being the bf16 post-conv activation
    matrix the GDN step consumed."""
    mixed = mixed_qkv.cpu()
    cstate = conv_state.cpu().clone()
    indices_c, cu_c, accepted_c = indices.cpu().long(), cu.cpu().long(), accepted.cpu().long()
    width = indices_c.shape[1]
    cols = cstate.shape[-1]
    post = mixed.clone()
    gdn_accepted = accepted_c.clone()
    for r in range(indices_c.shape[0]):
        bos, eos = int(cu_c[r]), int(cu_c[r + 1])
        n = eos - bos
        acc = int(accepted_c[r])
        source = int(indices_c[r, acc - 1]) if 1 <= acc <= width else 0
        conv_slot = int(indices_c[r, 0])
        offset = acc - 1
        if n <= 0 or source <= 0 or n > width:
            continue  # expected_decode treats it as invalid on its own
        if conv_slot <= 0 or offset + 2 > cols - 1 or (cols > n and offset > n - 1):
            gdn_accepted[r] = 0  # invalid: zero outputs, no writes
            continue
        y, new_state = conv_oracle.conv_update_tokens(
            mixed[bos:eos], cstate[conv_slot], conv_weight.cpu(),
            None if conv_bias is None else conv_bias.cpu(), offset)
        post[bos:eos] = y
        cstate[conv_slot] = new_state
    result = expected_decode(post, a, b, a_log, dt_bias, indices, cu, gdn_accepted.to(torch.int32),
                             pool, gate, weight, out, eps, return_pre=return_pre)
    return result + (cstate, post)
