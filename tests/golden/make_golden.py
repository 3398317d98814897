"""Write golden vectors for the post-conv GDN by running the reference's own Torch function.

Run where the reference source is present (the GPU test machines do not have it):

    python tests/golden/make_golden.py [--reference /root/reference/python]

It imports `post_conv_gdn` from the reference's python/lightdelta/reference/gdn.py (torch
only) and stores inputs and outputs as .npz data next to this script; bf16 arrays are stored
as their uint16 bit patterns.  The vectors pin the fp32 op order and the two bf16 rounding
points of the reference's math (gdn.py:116 and :120), which no closed form does.

Cases:
  scalar      the 1-element known-answer case of the reference's tests/test_gdn.py:47-55
  prefix      fp32, B=3 T=4 Hk=2 Hv=6 K=5 V=7, lengths [4,2,0], checkpoints (test_gdn.py:7-44)
  tiny_bf16   bf16, B=3 T=3 Hk=2 Hv=4 K=V=16, lengths [3,1,0], bf16 dt_bias / norm weight
  cfg1_step   1 step, B=1 Hk=4 Hv=8 K=V=128, the workload distributions listed below
  cfg1_64     64 consecutive single-token steps of cfg1 shapes, state carried across steps
  mtp         bf16, B=4 T=4 Hk=2 Hv=4 K=V=32, lengths [4,3,1,0], checkpoints
Workload distributions (seed 0): q,k,v,gate bf16 ~ N(0,1); a, b bf16 ~ N(0,1); A_log fp32
~ U(-1,1); dt_bias fp32 zeros; norm weight fp32 1 + 0.1 N(0,1); state fp32 ~ 0.02 N(0,1).
"""

from __future__ import annotations

import argparse
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def save(name: str, **arrays) -> None:
    out = {}
    for key, value in arrays.items():
        if isinstance(value, torch.Tensor):
            out[key] = bits(value)
            if value.dtype == torch.bfloat16:
                out[key + "__bf16"] = np.array(1)
        else:
            out[key] = np.asarray(value)
    np.savez_compressed(HERE / f"{name}.npz", **out)
    print(f"wrote {name}.npz")


def workload_inputs(gen, batch, tokens, hk, hv, dim, dtype=torch.bfloat16):
    def normal(*shape):
        return torch.randn(*shape, generator=gen)

    return dict(
        q=normal(batch, tokens, hk, dim).to(dtype),
        k=normal(batch, tokens, hk, dim).to(dtype),
        v=normal(batch, tokens, hv, dim).to(dtype),
        a=normal(batch, tokens, hv).to(dtype),
        b=normal(batch, tokens, hv).to(dtype),
        a_log=torch.rand(hv, generator=gen) * 2 - 1,
        dt_bias=torch.zeros(hv),
        gate=normal(batch, tokens, hv, dim).to(dtype),
        norm_weight=1 + 0.1 * normal(dim),
    )


FIELDS = ("q", "k", "v", "a", "b", "a_log", "dt_bias", "gate", "norm_weight")


def main() -> None:
    parser = argparse.ArgumentParser()
    parser.add_argument("--reference", default="/root/reference/python")
    args = parser.parse_args()
    sys.path.insert(0, args.reference)
    from lightdelta.reference import GDNInputs, post_conv_gdn  # the reference's own code

    def call(inp, state, lengths, **kw):
        return post_conv_gdn(GDNInputs(*(inp[f] for f in FIELDS)), state, lengths, **kw)

    # scalar known-answer case
    one = torch.ones(1, 1, 1, 1)
    zero = torch.zeros(1, 1, 1)
    inp = dict(q=one, k=one, v=one * 3, a=zero, b=zero, a_log=torch.zeros(1),
               dt_bias=torch.zeros(1), gate=one, norm_weight=torch.ones(1))
    r = call(inp, one * 2, torch.ones(1, dtype=torch.int32))
    save("scalar", state=one * 2, lengths=np.array([1]), output=r.output,
         final_state=r.final_state, **inp)

    # prefix case, fp32
    torch.manual_seed(7)
    batch, tokens, hk, hv, k, v = 3, 4, 2, 6, 5, 7
    rand = lambda *shape: torch.randn(shape)  # noqa: E731
    inp = dict(q=rand(batch, tokens, hk, k), k=rand(batch, tokens, hk, k),
               v=rand(batch, tokens, hv, v), a=rand(batch, tokens, hv), b=rand(batch, tokens, hv),
               a_log=rand(hv), dt_bias=rand(hv), gate=rand(batch, tokens, hv, v), norm_weight=rand(v))
    state = rand(batch, hv, v, k)
    lengths = torch.tensor([4, 2, 0])
    r = call(inp, state, lengths, save_checkpoints=True)
    save("prefix", state=state, lengths=lengths.numpy(), output=r.output,
         final_state=r.final_state, checkpoints=r.checkpoints, **inp)

    # tiny bf16 with bf16 dt_bias / weight
    gen = torch.Generator().manual_seed(1)
    inp = workload_inputs(gen, 3, 3, 2, 4, 16)
    inp["dt_bias"] = torch.randn(4, generator=gen).to(torch.bfloat16)
    inp["norm_weight"] = inp["norm_weight"].to(torch.bfloat16)
    state = 0.1 * torch.randn(3, 4, 16, 16, generator=gen)
    lengths = torch.tensor([3, 1, 0], dtype=torch.int32)
    r = call(inp, state, lengths, save_checkpoints=True, norm_eps=1e-5)
    save("tiny_bf16", state=state, lengths=lengths.numpy(), eps=np.array(1e-5),
         output=r.output, final_state=r.final_state, checkpoints=r.checkpoints, **inp)

    # cfg1: one step and 64 consecutive steps
    gen = torch.Generator().manual_seed(0)
    state0 = 0.02 * torch.randn(1, 8, 128, 128, generator=gen)
    steps = [workload_inputs(gen, 1, 1, 4, 8, 128) for _ in range(64)]
    for s in steps[1:]:  # per-layer parameters are fixed across steps
        for f in ("a_log", "dt_bias", "norm_weight"):
            s[f] = steps[0][f]
    lengths = torch.ones(1, dtype=torch.int32)
    r = call(steps[0], state0, lengths)
    save("cfg1_step", state=state0, lengths=lengths.numpy(), output=r.output,
         final_state=r.final_state, **steps[0])
    state = state0
    outputs = []
    for s in steps:
        r = call(s, state, lengths)
        outputs.append(r.output)
        state = r.final_state
    stacked = {f: torch.cat([s[f] for s in steps], 1) for f in ("q", "k", "v", "a", "b", "gate")}
    save("cfg1_64", state=state0, lengths=lengths.numpy(), output=torch.cat(outputs, 1),
         final_state=state, a_log=steps[0]["a_log"], dt_bias=steps[0]["dt_bias"],
         norm_weight=steps[0]["norm_weight"], **stacked)

    # MTP-shaped multi-token case with checkpoints
    gen = torch.Generator().manual_seed(2)
    inp = workload_inputs(gen, 4, 4, 2, 4, 32)
    state = 0.02 * torch.randn(4, 4, 32, 32, generator=gen)
    lengths = torch.tensor([4, 3, 1, 0], dtype=torch.int32)
    r = call(inp, state, lengths, save_checkpoints=True)
    save("mtp", state=state, lengths=lengths.numpy(), output=r.output,
         final_state=r.final_state, checkpoints=r.checkpoints, **inp)


if __name__ == "__main__":
    main()
