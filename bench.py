"""Benchmark of the fused GDN decode step on one MI355X.

Workload (the headline configuration): one Qwen3-Next-shape GDN decode layer, batch 32,
16 qk heads / 32 v heads, dk = dv = 128, bf16 activations, fp32 state pool of 256 slots x
32 heads x 128 x 128 (2 MiB per slot); batch rows map to random distinct slot ids and the
state is updated in place for consecutive steps.  A step is one `torch.ops.lightdelta.decode`
launch over the batch.

  python bench.py [--steps K] [--warmup W] [--gpus 1]

Timed region: K steps captured in one HIP graph and replayed once, bracketed by
torch.cuda.synchronize(); inputs are resident in HBM before it starts.  Printed: ONE JSON
line with steps/s (`value`), tokens/s, the roofline of the decode kernel and a CPU
baseline.

Roofline: algorithmic bytes per launch = B * HV * 128 * 128 * 4 B * 2 (read + write of every
state tile) = 134,217,728 B; `achieved` divides that by the average duration of one launch
in the timed region (HIP events on the launch stream around the K back-to-back graph
launches, so inter-kernel gaps count against it).  `traffic` (HBM bytes per launch from
rocprofv3 FETCH_SIZE + WRITE_SIZE, scaled by the counters' reading on a plain copy of known
size) is read from profiles/gdn_decode_b32_traffic.json when that measurement exists.
The headline runs the "keep" state cache policy: the 64 MiB working set of one layer stays
in the 256 MB Infinity Cache between consecutive steps.  A second, cache-cold figure rotates
16 disjoint slot sets through a 1024-slot (2 GiB) pool with the "stream" policy
(non-temporal state traffic), the regime of a many-layer model.

Further figures in the same line: `conv_fused` (the same step with the width-4 causal
conv1d + SiLU fused in front), `prefill` (32 x 1024, 1 x 4096 and 1024 x 32 tokens, both
algorithms), `mtp_verify` (B=64, T=4 verify plus the commit at a random accepted length), `copies`
(gather / scatter / slot-to-slot copy of 128 random pairs in a 1024-slot pool, and the bf16
conv pool) and `stack48` (48 layers captured as one HIP graph, batch 128, 1024 slots per
layer = 96 GiB of state, slot ids reshuffled before every replay, 256 replays timed end to
end; --no-stack skips it).

CPU baseline: the reference's packed Torch path (index_select gather, unfused GDN,
index_copy_ write-back; oracle/decode.py) on the host cores at the same shapes, timed for a
bounded number of steps.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "GDN decode steps/s + achieved HBM TB/s on state R/W, B=32, 32 v-heads"
BATCH, H, HV, DIM, POOL = 32, 16, 32, 128, 256
STATE_BYTES = BATCH * HV * DIM * DIM * 4 * 2  # one read + one write per state tile
HBM_PEAK_GBS = 8000.0
ORDER = ("qkv", "a", "b", "a_log", "dt_bias", "slots", "cu", "accepted", "pool", "gate",
         "weight", "out")
TRAFFIC_FILE = ROOT / "profiles" / "gdn_decode_b32_traffic.json"


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=64)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--cpu-seconds", type=float, default=15.0,
                   help="bound on the CPU-baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-cold", action="store_true")
    p.add_argument("--no-conv", action="store_true")
    p.add_argument("--no-stack", action="store_true",
                   help="skip the 48-layer, 96 GiB stack measurement")
    p.add_argument("--stack-steps", type=int, default=256)
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--no-mtp", action="store_true", help="skip the B=64, T=4 verify + commit")
    p.add_argument("--no-copies", action="store_true", help="skip the state-pool copy kernels")
    p.add_argument("--no-graph", action="store_true",
                   help="time K eager launches instead of one K-step graph replay")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="only run the plain slot-copy kernel (64 MiB read + 64 MiB write per "
                        "launch) K times, for scaling rocprofv3 byte counters")
    return p.parse_args()


def events():
    import torch

    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def capture(fn, steps):
    """One HIP graph holding `steps` calls of fn (warmed up on a side stream first)."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(steps):
            fn()
    return graph


def per_launch_us(fn, launches):
    """Mean / median kernel duration from HIP events around each eager launch."""
    import torch

    pairs = [events() for _ in range(launches)]
    for start, end in pairs:
        start.record()
        fn()
        end.record()
    torch.cuda.synchronize()
    times = sorted(s.elapsed_time(e) * 1000.0 for s, e in pairs)
    return sum(times) / len(times), times[len(times) // 2]


def timed_replay(graph):
    import torch

    start, end = events()
    torch.cuda.synchronize()
    start.record()
    graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1000.0


def cpu_baseline(seconds: float) -> dict:
    """The reference Torch path on the host CPU, same shapes, bounded sample."""
    import torch

    from lightdelta_amd.workloads import decode_case
    from oracle.decode import packed_reference_step

    threads = torch.get_num_threads()
    case = decode_case(BATCH, 1, num_k_heads=H, num_v_heads=HV, pool_slots=POOL, seed=0,
                       device="cpu")
    scratch = case["pool"].new_empty((1 + BATCH, *case["pool"].shape[1:]))
    args = [case[k] for k in ORDER]
    packed_reference_step(*args, 1e-6, scratch=scratch)  # warm-up
    times = []
    deadline = time.perf_counter() + seconds
    while len(times) < 3 or (time.perf_counter() < deadline and len(times) < 2000):
        t0 = time.perf_counter()
        packed_reference_step(*args, 1e-6, scratch=scratch)
        times.append(time.perf_counter() - t0)
    times.sort()
    median = times[len(times) // 2]
    cpu = platform.processor() or platform.machine()
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(1.0 / median, 3),
        "unit": "steps/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{len(times)} steps of the packed Torch reference path (index_select gather, "
                  f"unfused GDN, index_copy_ write-back) at B=32, 16/32 heads, 256-slot pool; "
                  f"median step {median * 1e3:.1f} ms; {cpu}",
    }


def conv_fused(case, op_args, steps, device):
    """The same step with the causal conv1d (width 4, SiLU, conv state of 3 columns, bf16
    pool of 256 slots x 8192 channels) fused in front: one decode_conv launch per step on the
    pre-conv activations."""
    import torch

    conv_dim = case["qkv"].shape[1]
    gen = torch.Generator().manual_seed(1)
    conv_state = torch.randn(POOL, conv_dim, 3, generator=gen).bfloat16().to(device)
    conv_weight = (torch.randn(conv_dim, 4, generator=gen) / 2).bfloat16().to(device)
    rest = op_args[1:]
    step = lambda: torch.ops.lightdelta.decode_conv(  # noqa: E731
        case["qkv"], conv_state, conv_weight, None, *rest, 1e-6)
    for _ in range(4):
        step()
    graph = capture(step, steps)
    graph.replay()
    torch.cuda.synchronize()
    elapsed = timed_replay(graph)
    rate = steps / elapsed
    conv_bytes = BATCH * conv_dim * 3 * 2 * 2  # conv state columns read + written
    return {
        "workload": "same step with the width-4 causal conv1d + SiLU fused in front "
                    "(bf16 conv pool 256 x 8192 x 3, no bias)",
        "steps_per_s": round(rate, 1),
        "us_per_step": round(elapsed * 1e6 / steps, 3),
        "state_TBps": round(STATE_BYTES * rate / 1e12, 3),
        "frac": round((STATE_BYTES + conv_bytes) * rate / 1e9 / HBM_PEAK_GBS, 4),
    }


def prefill(device):
    """Prefill of 32 prompts x 1024 tokens, of one 4096-token prompt and of 1024 prompts x 32
    tokens (16 qk / 32 v heads, states from pool slots), timed over a few eager launches
    each, under both algorithms (token-serial recurrence; 64-token chunks in the WY form on
    the matrix cores); `auto_selects` is the form the default picks."""
    import torch

    from lightdelta_amd import _lib, ops

    order = ("qkv", "a", "b", "a_log", "dt_bias", "slots", "has_initial", "cu_seqlens",
             "pool", "gate", "weight", "out")
    gen = torch.Generator(device=device).manual_seed(7)
    qkv_cols = (2 * H + HV) * DIM
    result = {}
    saved = ops.prefill_algorithm()
    for label, seqs, length in (("batch_32x1024", 32, 1024), ("single_4096", 1, 4096),
                                ("short_1024x32", 1024, 32)):
        total = seqs * length
        qkvz = torch.randn(total, qkv_cols + HV * DIM, generator=gen, device=device).bfloat16()
        ba = torch.randn(total, 2 * HV, generator=gen, device=device).bfloat16()
        case = dict(
            qkv=qkvz[:, :qkv_cols], a=ba[:, HV:], b=ba[:, :HV],
            a_log=torch.rand(HV, generator=gen, device=device) * 2 - 1,
            dt_bias=torch.zeros(HV, device=device),
            slots=torch.arange(1, seqs + 1, dtype=torch.int32, device=device),
            has_initial=torch.ones(seqs, dtype=torch.bool, device=device),
            cu_seqlens=torch.arange(0, total + 1, length, dtype=torch.int32, device=device),
            pool=torch.empty(seqs + 1, HV, DIM, DIM, device=device).normal_(0.0, 0.02,
                                                                            generator=gen),
            gate=qkvz[:, qkv_cols:].view(total, HV, DIM),
            weight=1 + 0.1 * torch.randn(DIM, generator=gen, device=device),
            out=torch.empty(total, HV, DIM, dtype=torch.bfloat16, device=device),
        )
        run = lambda: torch.ops.lightdelta.prefill(*[case[k] for k in order], 1e-6)  # noqa: E731
        entry = {"auto_selects": "chunked" if _lib.load().ld_gdn_prefill_auto_chunked(
            total, seqs, HV) else "token_serial"}
        try:
            for algorithm in ("token_serial", "chunked"):
                ops.set_prefill_algorithm(algorithm)
                run()
                torch.cuda.synchronize()
                start, end = events()
                reps = 5
                start.record()
                for _ in range(reps):
                    run()
                end.record()
                torch.cuda.synchronize()
                ms = start.elapsed_time(end) / reps
                entry[algorithm] = {"ms": round(ms, 3), "tokens_per_s": round(total / ms * 1e3, 1)}
                if algorithm == "chunked":
                    # matrix-core work of the WY form per (64-token chunk, v-head): the scan's
                    # 3,584 fp32 16x16x4 products and the prep's 640 fp32 16x16x4 (forward
                    # substitution) and 80 bf16 16x16x32 ones (the q.k and k.k tiles)
                    chunk_flop = (3584 + 640) * 2048 + 80 * 16384
                    flop = seqs * -(-length // 64) * HV * chunk_flop
                    entry[algorithm]["mfma_TFLOPs"] = round(flop / ms / 1e9, 1)
        finally:
            ops.set_prefill_algorithm(saved)
        result[label] = entry
        del case
    result["workload"] = ("prefill (state from the slot, recurrence over the prompt, gated "
                          "RMSNorm, final state to the slot), 16 qk / 32 v heads")
    return result


def copies(device):
    """State-pool copy kernels alone: a 1024-slot fp32 pool (32 x 128 x 128 per slot, 2 MiB)
    and a bf16 conv pool (4 x 8192 per slot, 64 KiB); 128 random (src, dst) pairs with
    padding slots (-1) among them.  gather_state into a packed buffer, scatter_state back,
    copy_state slot to slot, and the conv pool's gather_slots / scatter_slots, each timed
    as one HIP graph of 50 launches (launch overhead out of the figure).  Bytes are the rows
    each kernel actually reads plus the rows it writes (a gather writes zeros for padding
    rows)."""
    import torch

    ops = torch.ops.lightdelta
    gen = torch.Generator(device=device).manual_seed(11)
    slots_n, pairs = 1024, 128
    pool = torch.empty(slots_n, HV, DIM, DIM, device=device).normal_(generator=gen)
    conv = torch.empty(slots_n, 4, 8192, device=device).normal_(generator=gen).bfloat16()
    perm = torch.randperm(slots_n - 1, generator=gen, device=device)[: 2 * pairs] + 1
    src, dst = perm[:pairs].int(), perm[pairs:].int()
    src[::16] = -1
    dst[5::16] = -1
    valid = torch.ones(pairs, dtype=torch.bool, device=device)
    packed = torch.empty(pairs, HV, DIM, DIM, device=device)
    packed_conv = torch.empty(pairs, 4, 8192, dtype=torch.bfloat16, device=device)
    n_src = int((src > 0).sum())
    n_dst = int((dst > 0).sum())
    n_both = int(((src > 0) & (dst > 0)).sum())
    row, conv_row = HV * DIM * DIM * 4, 4 * 8192 * 2
    runs = {
        "gather_state": (lambda: ops.gather_state(pool, src, valid, packed), (n_src + pairs) * row),
        "scatter_state": (lambda: ops.scatter_state(packed, dst, pool), 2 * n_dst * row),
        "copy_state": (lambda: ops.copy_state(pool, src, dst), 2 * n_both * row),
        "gather_slots_conv": (lambda: ops.gather_slots(conv, src, valid, packed_conv),
                              (n_src + pairs) * conv_row),
        "scatter_slots_conv": (lambda: ops.scatter_slots(packed_conv, dst, conv),
                               2 * n_dst * conv_row),
    }
    result = {}
    launches = 50
    for name, (fn, nbytes) in runs.items():
        graph = capture(fn, launches)
        graph.replay()
        us = timed_replay(graph) / launches * 1e6
        result[name] = {"us": round(us, 2), "bytes": nbytes, "TBps": round(nbytes / us / 1e6, 3)}
        del graph
    result["workload"] = ("state-pool copies alone: 1024-slot fp32 pool (2 MiB per slot) and "
                          "bf16 conv pool (64 KiB per slot), 128 random pairs with padding -1")
    del pool, conv, packed, packed_conv
    return result


def mtp_verify(steps, device):
    """MTP speculative verify at B = 64, T = 4 (1 accepted + 3 draft tokens per sequence),
    16 qk / 32 v heads, then the commit.  Sequence r owns a home slot and 3 scratch slots;
    the verify step reads the state from the home slot and writes the 4 per-token states to
    [home, s1, s2, s3]; the commit copies the state at a random accepted length a in [1, 4]
    back to the home slot (copy_state from s_(a-1); nothing when a = 1).  `steps`
    (verify, commit) pairs, each with its own accepted lengths drawn on the device
    beforehand, are captured as one HIP graph and replayed once, timed end to end; the
    verify launches alone are also timed per launch (HIP events)."""
    import torch

    from lightdelta_amd.workloads import decode_case

    batch, width = 64, 4
    order = ("qkv", "a", "b", "a_log", "dt_bias", "slots", "cu", "accepted", "pool", "gate",
             "weight", "out")
    case = decode_case(batch, width, num_k_heads=H, num_v_heads=HV, pool_slots=batch * width + 2,
                       seed=5, device=device)
    case["accepted"].fill_(1)  # the verify starts from slot[r, 0], the home slot
    slots = case["slots"]
    gen = torch.Generator(device=device).manual_seed(12)
    accepted = torch.randint(1, width + 1, (steps, batch), generator=gen, device=device)
    src = torch.gather(slots.long().expand(steps, -1, -1), 2, (accepted - 1).unsqueeze(2))[..., 0]
    src = torch.where(accepted > 1, src, torch.full_like(src, -1)).int()
    dst = torch.where(accepted > 1, slots[:, 0].long().expand(steps, -1),
                      torch.full_like(src, -1, dtype=torch.long)).int()
    args = [case[k] for k in order]
    verify = lambda: torch.ops.lightdelta.decode(*args, 1e-6)  # noqa: E731
    verify()
    torch.cuda.synchronize()
    verify_mean, verify_median = per_launch_us(verify, 50)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        verify()
        torch.ops.lightdelta.copy_state(case["pool"], src[0], dst[0])
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for step in range(steps):
            verify()
            torch.ops.lightdelta.copy_state(case["pool"], src[step], dst[step])
    graph.replay()  # warm-up replay
    seconds = timed_replay(graph)
    step_us = seconds / steps * 1e6
    verify_bytes = batch * HV * 65536 * (1 + width)
    commit_bytes = int((accepted > 1).sum()) * HV * 65536 * 2 // steps
    return {
        "workload": ("MTP verify B=64, T=4, 16 qk / 32 v heads, per-token states to "
                     "[home, s1, s2, s3], then commit at a random accepted length (copy_state)"),
        "us_per_step": round(step_us, 2),
        "steps_per_s": round(1e6 / step_us, 1),
        "tokens_per_s": round(batch * width * 1e6 / step_us, 1),
        "verify_us": round(verify_mean, 2),
        "verify_median_us": round(verify_median, 2),
        "verify_TBps": round(verify_bytes / verify_mean / 1e6, 3),
        "commit_bytes_per_step": commit_bytes,
        "step_TBps": round((verify_bytes + commit_bytes) / step_us / 1e6, 3),
        "frac": round((verify_bytes + commit_bytes) / step_us / 1e3 / HBM_PEAK_GBS, 4),
    }


def stack48(steps, device):
    """48 GDN decode layers captured as one HIP graph, batch 128, 16 qk / 32 v heads, 1024
    slots per layer (96 GiB fp32 state), stream cache policy; the slot ids (shared by every
    layer) are reshuffled before every replay by a device-to-device copy from a table of
    random distinct ids.  `steps` replays are timed end to end, reshuffles included."""
    import torch

    from lightdelta_amd import ops
    from lightdelta_amd.workloads import stack_case, stack_layer

    layers_n, batch, slots_n = 48, 128, 1024
    case = stack_case(layers_n, batch, pool_slots=slots_n, seed=5, device=device)
    layers = [stack_layer(case, layer) for layer in range(layers_n)]

    def step():
        for a in layers:
            torch.ops.lightdelta.decode(*[a[k] for k in ORDER], 1e-6)

    policy = ops.state_cache_policy()
    ops.set_state_cache_policy("stream")
    try:
        step()
        graph = capture(step, 1)
    finally:
        ops.set_state_cache_policy(policy)
    gen = torch.Generator().manual_seed(6)
    table = torch.stack([torch.randperm(slots_n - 1, generator=gen)[:batch] + 1
                         for _ in range(steps)]).to(torch.int32).view(steps, batch, 1).to(device)
    for i in range(2):  # untimed warm-up replays
        case["slots"].copy_(table[i])
        graph.replay()
    torch.cuda.synchronize()
    start, end = events()
    start.record()
    for i in range(steps):
        case["slots"].copy_(table[i])
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    elapsed = start.elapsed_time(end) / 1000.0
    step_bytes = layers_n * batch * HV * DIM * DIM * 4 * 2
    rate = steps / elapsed
    return {
        "workload": "48-layer stack of decode steps in one HIP graph, batch 128, 16 qk / 32 v "
                    "heads, 1024 slots per layer (96 GiB fp32 state), slot ids reshuffled "
                    "before every replay, stream cache policy",
        "steps": steps,
        "ms_per_step": round(elapsed * 1000.0 / steps, 4),
        "steps_per_s": round(rate, 2),
        "tokens_per_s": round(rate * batch, 1),
        "state_bytes_per_step": step_bytes,
        "state_TBps": round(step_bytes * rate / 1e12, 3),
        "frac": round(step_bytes * rate / 1e9 / HBM_PEAK_GBS, 4),
    }


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}); this build has no "
              "multi-GPU path -- the op needs no cross-GPU exchange and shards by slots or "
              "heads outside it.", file=sys.stderr)
        sys.exit(2)

    import torch

    import lightdelta_amd  # noqa: F401  (registers torch.ops.lightdelta)
    from lightdelta_amd import _lib, ops
    from lightdelta_amd.workloads import decode_case

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    _lib.load()
    device = torch.device("cuda:0")
    torch.manual_seed(0)

    if args.calibrate_copy:
        pool = torch.empty(2 * BATCH + 1, HV, DIM, DIM, device=device).normal_()
        src = torch.arange(1, BATCH + 1, device=device, dtype=torch.int32)
        dst = src + BATCH
        copy = lambda: torch.ops.lightdelta.copy_state(pool, src, dst)  # noqa: E731
        for _ in range(args.warmup):
            copy()
        mean_us, median_us = per_launch_us(copy, args.steps)
        print(json.dumps({"calibration": "copy_state", "bytes_read": STATE_BYTES // 2,
                          "bytes_written": STATE_BYTES // 2, "launches": args.steps,
                          "mean_us": round(mean_us, 3),
                          "achieved_GBps": round(STATE_BYTES / mean_us / 1e3, 1)}))
        return

    case = decode_case(BATCH, 1, num_k_heads=H, num_v_heads=HV, pool_slots=POOL, seed=0,
                       device=device)
    op_args = [case[k] for k in ORDER]
    step = lambda: torch.ops.lightdelta.decode(*op_args, 1e-6)  # noqa: E731
    # one layer stepped in place: its 64 MiB stay in the Infinity Cache between steps
    ops.set_state_cache_policy("keep")

    for _ in range(args.warmup):
        step()
    if args.no_graph:
        torch.cuda.synchronize()
        start, end = events()
        start.record()
        for _ in range(args.steps):
            step()
        end.record()
        torch.cuda.synchronize()
        elapsed = start.elapsed_time(end) / 1000.0
    else:
        graph = capture(step, args.steps)
        graph.replay()  # upload + warm the graph (untimed)
        torch.cuda.synchronize()
        elapsed = timed_replay(graph)  # exactly K steps
    ms_per_step = elapsed * 1000.0 / args.steps
    steps_per_s = args.steps / elapsed

    launch_us = elapsed * 1e6 / args.steps
    achieved = STATE_BYTES / (launch_us * 1e-6) / 1e9
    traffic = None
    if TRAFFIC_FILE.exists():
        traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")

    result = {
        "metric": METRIC,
        "value": round(steps_per_s, 1),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "GDN decode layer, B=32, 16 qk / 32 v heads, dk=dv=128, bf16 "
                        "activations, fp32 state pool 256 x 32 x 128 x 128, random distinct "
                        "slots, in-place consecutive steps, "
                        + ("eager launches" if args.no_graph else "HIP-graph replay"),
            "batch": BATCH, "qk_heads": H, "v_heads": HV, "head_dim": DIM, "pool_slots": POOL,
        },
        "tokens_per_s": round(steps_per_s * BATCH, 1),
        "state_TBps": round(STATE_BYTES * steps_per_s / 1e12, 3),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "gdn_decode_kernel",
            "kernel_mean_us": round(launch_us, 3),
            "algorithmic_bytes": STATE_BYTES,
            "cache_policy": ops.state_cache_policy(),
        },
    }

    if not args.no_cold:
        # Cache-cold variant: 16 disjoint slot sets rotated through a 1024-slot pool.
        big = torch.empty(1024, HV, DIM, DIM, device=device).normal_(0.0, 0.02)
        perm = torch.randperm(1023, device=device)[: 16 * BATCH] + 1
        sets = [perm[i * BATCH:(i + 1) * BATCH].to(torch.int32).view(BATCH, 1) for i in range(16)]
        cold_args = list(op_args)
        cold_args[ORDER.index("pool")] = big

        def cold_pass():
            for slots in sets:
                cold_args[ORDER.index("slots")] = slots
                torch.ops.lightdelta.decode(*cold_args, 1e-6)

        keep_policy = ops.state_cache_policy()
        ops.set_state_cache_policy("stream")
        cold_graph = capture(cold_pass, max(1, args.steps // 16))
        ops.set_state_cache_policy(keep_policy)
        cold_graph.replay()
        cold_elapsed = timed_replay(cold_graph)
        cold_steps = 16 * max(1, args.steps // 16)
        cold_rate = cold_steps / cold_elapsed
        result["cold"] = {
            "workload": "same step, 16 disjoint slot sets rotated through a 1024-slot (2 GiB) "
                        "pool; working set exceeds the 256 MB Infinity Cache",
            "cache_policy": "stream",
            "steps_per_s": round(cold_rate, 1),
            "state_TBps": round(STATE_BYTES * cold_rate / 1e12, 3),
            "frac": round(STATE_BYTES * cold_rate / 1e9 / HBM_PEAK_GBS, 4),
        }
        del big

    if not args.no_conv:
        result["conv_fused"] = conv_fused(case, op_args, args.steps, device)

    if not args.no_prefill:
        result["prefill"] = prefill(device)

    if not args.no_mtp:
        result["mtp_verify"] = mtp_verify(args.steps, device)

    if not args.no_copies:
        result["copies"] = copies(device)

    if not args.no_stack:
        case = op_args = graph = None  # noqa: F841  (release the B=32 pools first)
        torch.cuda.empty_cache()
        result["stack48"] = stack48(args.stack_steps, device)

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
