"""Benchmark of the fused GDN decode step on one MI355X.

Workload (the headline configuration): one Qwen3-Next-shape GDN decode layer, batch 32,
16 qk heads / 32 v heads, dk = dv = 128, bf16 activations, fp32 state pool of 256 slots x
32 heads x 128 x 128 (2 MiB per slot); batch rows map to random distinct slot ids and the
state is updated in place for consecutive steps.  A step is one `torch.ops.lightdelta.decode`
launch over the batch.

  python bench.py [--steps K] [--warmup W] [--gpus 1]

Timed region: K steps captured in one HIP graph; each replay is bracketed by
torch.cuda.synchronize() and timed with HIP events, and the figure is the median of 30 such
replays (--samples), with their spread beside it; inputs are resident in HBM before it
starts.  Printed: ONE JSON line with steps/s (`value`), tokens/s, the roofline of the decode
kernel and a CPU baseline.

Roofline: algorithmic bytes per launch = B * HV * 128 * 128 * 4 B * 2 (read + write of every
state tile) = 134,217,728 B; `achieved` divides that by the average duration of one launch
in the timed region (HIP events on the launch stream around the K back-to-back graph
launches of the median replay, so inter-kernel gaps count against it).  `traffic` (HBM bytes per launch from
rocprofv3 FETCH_SIZE + WRITE_SIZE, scaled by the counters' reading on a plain copy of known
size) is read from profiles/gdn_decode_b32_traffic.json when that measurement exists.
The headline runs the "keep" state cache policy: the 64 MiB working set of one layer stays
in the 256 MB Infinity Cache between consecutive steps.  A second, cache-cold figure rotates
16 disjoint slot sets through a 1024-slot (2 GiB) pool with the "stream" policy
(non-temporal state traffic), the regime of a many-layer model.

Further figures in the same line:
  conv_fused      the step with the width-4 causal conv1d + SiLU fused in front: hot (B=32),
                  cold (slot sets rotated through 2048-slot pools) and a B=64, T=4 verify;
  config1         the first workload configuration (B=1, 4/8 heads, conv-fused, zero conv
                  state): graph and eager latency per step;
  operator_table  the reference's own operator benchmark (16/48 heads, B 1/4/8 x T 1-4,
                  eager "indexed" and HIP-graph medians, its method), beside its H100 medians;
  host_cost       host time of one eager GDNBackend call at B=1 and B=8;
  prefill         32 x 1024, 1 x 4096 and 1024 x 32 tokens under both algorithms;
  mtp_verify      B=64, T=4 verify plus the commit at a random accepted length (hot);
  mtp_verify_cold the same verify with slot sets rotated through a 4 GiB pool;
  copies          gather / scatter / slot-to-slot copy of 128 random pairs in a 1024-slot
                  pool, and the bf16 conv pool;
  stack48         48 layers captured as one HIP graph, batch 128, 1024 slots per layer =
                  96 GiB of state, slot ids reshuffled before every replay, 256 replays timed
                  end to end (--no-stack skips it);
  stack48_conv    the same stack of conv-fused steps (decode_conv, one launch per layer, each
                  layer with its own 1024-slot bf16 conv pool), the serving layer's step.

CPU baseline: the reference's packed Torch path (index_select gather, unfused GDN,
index_copy_ write-back; oracle/decode.py) on every host core this process may use, at the
headline shapes and at the first configuration (with torch's conv1d in front), timed on
bounded samples.
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
# The reference's published H100 operator medians (docs/performance.md:12-25 of the
# reference; 16/48 heads): (batch, tokens per request) -> (indexed us, graph us).
REF_H100_US = {  # (reference, fusion, indexed, graph) medians in us
    (1, 1): (983.09, 321.23, 17.47, 12.38), (1, 2): (1476.64, 313.04, 18.91, 14.11),
    (1, 3): (1781.74, 326.14, 21.22, 16.14), (1, 4): (2089.46, 313.46, 19.90, 19.17),
    (4, 1): (995.09, 307.68, 18.27, 14.72), (4, 2): (1525.97, 314.86, 19.73, 19.50),
    (4, 3): (1831.23, 313.06, 24.70, 24.48), (4, 4): (2111.70, 300.53, 30.46, 30.10),
    (8, 1): (1014.74, 375.63, 20.48, 20.21), (8, 2): (1797.76, 305.09, 31.98, 31.84),
    (8, 3): (1872.11, 312.96, 42.24, 42.29), (8, 4): (2117.74, 367.98, 53.73, 53.57),
}
# The reference benchmark's four configurations (configs/{reference,fusion,indexed,graph}.toml
# of the reference): compute, state access, graph replay.
OPERATOR_MODES = (("reference", "torch_reference", "packed", False),
                  ("fusion", "cuda_fused", "packed", False),
                  ("indexed", "cuda_fused", "indexed", False),
                  ("graph", "cuda_fused", "indexed", True))


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=64)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--samples", type=int, default=REPLAY_SAMPLES,
                   help="timed replays of the headline and cold graphs (median reported)")
    p.add_argument("--cpu-seconds", type=float, default=15.0,
                   help="bound on the CPU-baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-cold", action="store_true")
    p.add_argument("--no-tp", action="store_true",
                   help="skip the step at one GPU's share under head parallelism (TP = 2, 4)")
    p.add_argument("--no-conv", action="store_true")
    p.add_argument("--no-stack", action="store_true",
                   help="skip the 48-layer, 96 GiB stack measurement")
    p.add_argument("--stack-steps", type=int, default=256)
    p.add_argument("--no-stack-plain", action="store_true",
                   help="skip the post-conv 48-layer stack (keep the conv-fused one)")
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--no-mtp", action="store_true", help="skip the B=64, T=4 verify + commit")
    p.add_argument("--no-copies", action="store_true", help="skip the state-pool copy kernels")
    p.add_argument("--no-table", action="store_true",
                   help="skip the reference's operator table (16/48 heads, B 1-8, T 1-4) and "
                        "the host-cost figure")
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


# Timed replays per graph figure: the median is reported (the reference's benchmark takes the
# median of 30 samples, benchmarks/gdn.py:53-65,73).
REPLAY_SAMPLES = 30


def replay_median(graph, samples=REPLAY_SAMPLES):
    """Median seconds of `samples` timed replays of graph (each bracketed by
    synchronisations), and all the samples."""
    import statistics

    times = [timed_replay(graph) for _ in range(samples)]
    return statistics.median(times), times


def spread_us(times, units):
    """min / p10 / median / p90 / max of replay times, in us per unit (step or launch)."""
    ordered = sorted(t * 1e6 / units for t in times)
    pick = lambda q: ordered[min(len(ordered) - 1, int(q * len(ordered)))]  # noqa: E731
    return {"samples": len(ordered), "min": round(ordered[0], 3), "p10": round(pick(0.1), 3),
            "median": round(ordered[len(ordered) // 2] if len(ordered) % 2 else
                            (ordered[len(ordered) // 2 - 1] + ordered[len(ordered) // 2]) / 2, 3),
            "p90": round(pick(0.9), 3), "max": round(ordered[-1], 3)}


def _cpu_model() -> str:
    cpu = platform.processor() or platform.machine()
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return cpu


def _time_cpu(step, seconds, at_least=3, at_most=2000):
    """Median seconds per call of step() over a sample bounded by `seconds` of CPU time."""
    step()  # warm-up
    times = []
    deadline = time.perf_counter() + seconds
    while len(times) < at_least or (time.perf_counter() < deadline and len(times) < at_most):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_baseline(seconds: float) -> dict:
    """The reference's Torch path on the host CPU, timed on bounded samples of the same
    workloads: the packed path (index_select gather, unfused GDN, index_copy_ write-back;
    oracle/decode.py) at the headline configuration (B=32, 16/32 heads), and at B=1, 4/8
    heads with the width-4 causal conv (oracle/conv.py) in front.  Torch uses every core this
    process may run on (os.sched_getaffinity)."""
    import torch

    from lightdelta_amd.workloads import decode_case
    from oracle import conv as conv_oracle
    from oracle.decode import packed_reference_step

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    case = decode_case(BATCH, 1, num_k_heads=H, num_v_heads=HV, pool_slots=POOL, seed=0,
                       device="cpu")
    scratch = case["pool"].new_empty((1 + BATCH, *case["pool"].shape[1:]))
    args = [case[k] for k in ORDER]
    median, count = _time_cpu(lambda: packed_reference_step(*args, 1e-6, scratch=scratch),
                              seconds * 0.75)

    c1 = decode_case(1, 1, num_k_heads=4, num_v_heads=8, pool_slots=3, seed=0, device="cpu")
    conv_dim = c1["qkv"].shape[1]
    conv_state = torch.zeros(3, conv_dim, 3, dtype=torch.bfloat16)
    conv_weight = (torch.randn(conv_dim, 4, generator=torch.Generator().manual_seed(1)) / 2
                   ).bfloat16()
    pre_conv = c1["qkv"].clone()
    c1_args = [c1[k] for k in ORDER]
    c1_scratch = c1["pool"].new_empty((2, *c1["pool"].shape[1:]))

    def config1_step():  # conv through torch's conv1d (groups = channels), then the shift
        window = conv_state[1:2]
        c1_args[0] = conv_oracle.conv_update_reference_form(pre_conv, window, conv_weight)
        conv_state[1:2] = torch.cat([window[..., 1:], pre_conv[..., None]], -1)
        packed_reference_step(*c1_args, 1e-6, scratch=c1_scratch)

    median1, count1 = _time_cpu(config1_step, seconds * 0.25)
    return {
        "value": round(1.0 / median, 3),
        "unit": "steps/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{count} steps of the packed Torch reference path (index_select gather, "
                  f"unfused GDN, index_copy_ write-back) at B=32, 16/32 heads, 256-slot pool; "
                  f"median step {median * 1e3:.2f} ms; torch threads {cores}; {_cpu_model()}",
        "config1": {
            "value": round(1.0 / median1, 2),
            "unit": "steps/s",
            "us_per_step": round(median1 * 1e6, 1),
            "sample": f"{count1} steps at B=1, 4/8 heads: width-4 causal conv + SiLU from a "
                      f"zero conv state, then the packed Torch path",
        },
    }


def _graph_us(fn, steps, samples=REPLAY_SAMPLES):
    """us per call of `steps` calls of fn captured in one HIP graph: the median of `samples`
    timed replays."""
    import torch

    graph = capture(fn, steps)
    graph.replay()
    torch.cuda.synchronize()
    return replay_median(graph, samples)[0] * 1e6 / steps


def conv_fused(case, op_args, steps, device):
    """The step with the causal conv1d (width 4, SiLU, bf16 conv pool of 8192 channels, no
    bias) fused in front, one decode_conv launch per step on the pre-conv activations:
    `hot` (B=32, the same 32 slots, keep policy), `cold` (B=32, 16 disjoint slot sets
    rotated through 2048-slot SSM and conv pools, stream policy), `verify_b64_t4` (B=64,
    T=4 speculative verify with a 6-column conv state and random accepted counts, hot) and
    `verify_b64_t4_cold` (the same through 8 disjoint slot sets, stream policy)."""
    import torch

    from lightdelta_amd import ops
    from lightdelta_amd.workloads import decode_case

    conv_dim = case["qkv"].shape[1]
    gen = torch.Generator().manual_seed(1)
    conv_weight = (torch.randn(conv_dim, 4, generator=gen) / 2).bfloat16().to(device)
    saved = ops.state_cache_policy()
    result = {"workload": "decode_conv: width-4 causal conv1d + SiLU fused in front of the "
                          "GDN step, bf16 conv pool of 8192 channels, no bias"}
    try:
        ops.set_state_cache_policy("keep")
        conv_state = torch.randn(POOL, conv_dim, 3, generator=gen).bfloat16().to(device)
        rest = op_args[1:]
        hot = lambda: torch.ops.lightdelta.decode_conv(  # noqa: E731
            case["qkv"], conv_state, conv_weight, None, *rest, 1e-6)
        us = _graph_us(hot, steps)
        conv_bytes = BATCH * conv_dim * 3 * 2 * 2  # conv state columns read + written
        result["hot"] = {
            "us_per_step": round(us, 3), "steps_per_s": round(1e6 / us, 1),
            "state_TBps": round(STATE_BYTES / us / 1e6, 3),
            "frac": round((STATE_BYTES + conv_bytes) / us / 1e3 / HBM_PEAK_GBS, 4),
            "cache_policy": "keep"}
        del conv_state

        ops.set_state_cache_policy("stream")
        big = torch.empty(2049, HV, DIM, DIM, device=device).normal_(0.0, 0.02)
        big_conv = torch.zeros(2049, conv_dim, 3, dtype=torch.bfloat16, device=device)
        perm = torch.randperm(2048, device=device)[: 16 * BATCH] + 1
        sets = [perm[i * BATCH:(i + 1) * BATCH].to(torch.int32).view(BATCH, 1) for i in range(16)]
        cold_args = list(rest)
        pool_at, slots_at = ORDER.index("pool") - 1, ORDER.index("slots") - 1
        cold_args[pool_at] = big

        def cold_pass():
            for slots in sets:
                cold_args[slots_at] = slots
                torch.ops.lightdelta.decode_conv(case["qkv"], big_conv, conv_weight, None,
                                                 *cold_args, 1e-6)

        us = _graph_us(cold_pass, max(1, steps // 16)) / 16
        result["cold"] = {
            "us_per_step": round(us, 3), "steps_per_s": round(1e6 / us, 1),
            "frac": round((STATE_BYTES + conv_bytes) / us / 1e3 / HBM_PEAK_GBS, 4),
            "cache_policy": "stream"}
        del big, big_conv

        ops.set_state_cache_policy("keep")
        batch, width = 64, 4
        v = decode_case(batch, width, num_k_heads=H, num_v_heads=HV,
                        pool_slots=batch * width + 2, seed=5, device=device)
        v["accepted"].copy_(torch.randint(1, width + 1, (batch,), generator=gen).int())
        v_conv = torch.randn(batch * width + 2, conv_dim, 3 + width - 1, generator=gen
                             ).bfloat16().to(device)
        v_args = [v[k] for k in ORDER[1:]]
        verify = lambda: torch.ops.lightdelta.decode_conv(  # noqa: E731
            v["qkv"], v_conv, conv_weight, None, *v_args, 1e-6)
        us = _graph_us(verify, steps)
        v_bytes = batch * HV * 65536 * (1 + width) + batch * conv_dim * 6 * 2 * 2
        result["verify_b64_t4"] = {
            "us_per_step": round(us, 3), "tokens_per_s": round(batch * width * 1e6 / us, 1),
            "TBps": round(v_bytes / us / 1e6, 3), "cache_policy": "keep",
            "accepted": "random in 1..4 per request, conv state of 6 columns"}
        del v_conv

        # the same verify cache-cold: 8 disjoint slot sets rotated through 2049-slot pools
        ops.set_state_cache_policy("stream")
        big = torch.empty(2049, HV, DIM, DIM, device=device).normal_(0.0, 0.02)
        big_conv = torch.zeros(2049, conv_dim, 3 + width - 1, dtype=torch.bfloat16, device=device)
        perm = torch.randperm(2048, device=device)[: 8 * batch * width] + 1
        vsets = [perm[i * batch * width:(i + 1) * batch * width].to(torch.int32).view(batch, width)
                 for i in range(8)]
        cold_args = list(v_args)
        cold_args[pool_at] = big

        def verify_cold_pass():
            for s in vsets:
                cold_args[slots_at] = s
                torch.ops.lightdelta.decode_conv(v["qkv"], big_conv, conv_weight, None,
                                                 *cold_args, 1e-6)

        us = _graph_us(verify_cold_pass, max(1, steps // 8)) / 8
        result["verify_b64_t4_cold"] = {
            "us_per_step": round(us, 3), "tokens_per_s": round(batch * width * 1e6 / us, 1),
            "TBps": round(v_bytes / us / 1e6, 3), "frac": round(v_bytes / us / 1e3 / HBM_PEAK_GBS, 4),
            "cache_policy": "stream"}
        del big, big_conv
    finally:
        ops.set_state_cache_policy(saved)
    return result


def operator_table(device, iterations=30):
    """The reference's operator benchmark, same shapes and method (benchmarks/gdn.py:13-94 of
    the reference): 16 qk / 48 v heads, B in {1, 4, 8} x T in {1..4}, its seeded inputs
    (qkv and gate bf16 0.2 N(0,1), pool 0.1 N(0,1) over slots 1..B*T, bf16 dt_bias and norm
    weight), five warm-up calls on a side stream, then `iterations` samples that each restore
    the pool outside the timed interval and time one call with HIP events, for its four
    GDNBackend configurations: `reference` (the unfused Torch computation, packed state
    access), `fusion` (the fused kernel, packed state access), `indexed` (the fused kernel on
    the pool directly) -- all eager, host dispatch included -- and `graph` (the indexed call
    replayed from a HIP graph).  Medians in us, beside the reference's H100 medians
    (docs/performance.md:12-25 of the reference)."""
    import statistics

    import torch

    from lightdelta_amd import ops
    from lightdelta_amd.backend import GDNBackend
    from lightdelta_amd.config import BackendConfig

    saved = ops.state_cache_policy()
    ops.set_state_cache_policy("keep")  # the pool is restored (written) right before each call
    rows = {}
    try:
        for batch in (1, 4, 8):
            for width in (1, 2, 3, 4):
                torch.manual_seed(42)
                n = batch * width
                qkvz = torch.randn(n, 16384, device=device, dtype=torch.bfloat16) * 0.2
                ba = torch.randn(n, 96, device=device, dtype=torch.bfloat16)
                pool = torch.randn(n + 1, 48, 128, 128, device=device) * 0.1
                state = pool.clone()
                case = dict(
                    qkv=qkvz[:, :10240], a=ba[:, 48:], b=ba[:, :48],
                    a_log=torch.randn(48, device=device),
                    dt_bias=torch.randn(48, device=device, dtype=torch.bfloat16),
                    slots=torch.arange(1, n + 1, device=device, dtype=torch.int32).view(batch, width),
                    cu=torch.arange(0, n + 1, width, device=device, dtype=torch.int32),
                    accepted=torch.ones(batch, device=device, dtype=torch.int32),
                    pool=pool, gate=qkvz[:, 10240:].view(n, 48, 128),
                    weight=torch.randn(128, device=device, dtype=torch.bfloat16),
                    out=torch.empty(n, 48, 128, device=device, dtype=torch.bfloat16),
                )
                cell = {}
                for name, compute, state_io, replay in OPERATOR_MODES:
                    backend = GDNBackend(BackendConfig(compute=compute, state_io=state_io))
                    side = torch.cuda.Stream()
                    side.wait_stream(torch.cuda.current_stream())
                    with torch.cuda.stream(side):
                        for _ in range(5):
                            pool.copy_(state)
                            backend(**case)
                    torch.cuda.current_stream().wait_stream(side)
                    graph = None
                    if replay:
                        graph = torch.cuda.CUDAGraph()
                        with torch.cuda.graph(graph):
                            backend(**case)
                        execute = graph.replay
                    else:
                        execute = (lambda b: lambda: b(**case))(backend)
                    timers = []
                    for _ in range(iterations):
                        start, end = events()
                        pool.copy_(state)
                        start.record()
                        execute()
                        end.record()
                        timers.append((start, end))
                    torch.cuda.synchronize()
                    cell[f"{name}_us"] = round(statistics.median(
                        a.elapsed_time(b) * 1000 for a, b in timers), 2)
                    del graph, backend
                for (name, *_), h100 in zip(OPERATOR_MODES, REF_H100_US[(batch, width)]):
                    cell[f"h100_{name}_us"] = h100
                    cell[f"speedup_{name}"] = round(h100 / cell[f"{name}_us"], 2)
                rows[f"B{batch}_T{width}"] = cell
                del case, pool, state, qkvz, ba
    finally:
        ops.set_state_cache_policy(saved)
    # The same method on a one-kernel graph of a trivial torch op: what a HIP graph replay
    # costs on this platform before any work of ours.
    x = torch.zeros(1, device=device)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        x.add_(1)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        x.add_(1)
    timers = []
    for _ in range(iterations):
        start, end = events()
        start.record()
        graph.replay()
        end.record()
        timers.append((start, end))
    torch.cuda.synchronize()
    rows["graph_replay_floor_us"] = round(statistics.median(
        a.elapsed_time(b) * 1000 for a, b in timers), 2)
    rows["workload"] = ("the reference's operator benchmark: 16 qk / 48 v heads, its four "
                        "GDNBackend configurations (reference: Torch computation + packed state; "
                        "fusion: fused kernel + packed state; indexed: fused kernel on the pool; "
                        "all eager, host dispatch included; graph: the indexed call replayed from "
                        f"a HIP graph), median of {iterations} samples, pool restored outside "
                        "the timed interval; h100_* = the reference's published H100 medians; "
                        "graph_replay_floor_us = the replay of a one-kernel graph of torch's "
                        "x.add_(1), same method")
    return rows


def config1(device, steps):
    """The first workload configuration on the GPU: B=1, 4 qk / 8 v heads, the conv-fused
    step (width-4 conv from a zero conv state, SiLU) on one layer, `steps` consecutive
    in-place steps: graph replay (us per step) and eager calls (HIP events around each call,
    host dispatch included, median)."""
    import statistics

    import torch

    from lightdelta_amd.workloads import decode_case

    case = decode_case(1, 1, num_k_heads=4, num_v_heads=8, pool_slots=3, seed=0, device=device)
    conv_dim = case["qkv"].shape[1]
    conv_state = torch.zeros(3, conv_dim, 3, dtype=torch.bfloat16, device=device)
    conv_weight = (torch.randn(conv_dim, 4, generator=torch.Generator().manual_seed(1)) / 2
                   ).bfloat16().to(device)
    rest = [case[k] for k in ORDER[1:]]
    step = lambda: torch.ops.lightdelta.decode_conv(  # noqa: E731
        case["qkv"], conv_state, conv_weight, None, *rest, 1e-6)
    graph_us = _graph_us(step, steps)
    timers = []
    for _ in range(50):
        start, end = events()
        start.record()
        step()
        end.record()
        timers.append((start, end))
    torch.cuda.synchronize()
    eager = statistics.median(a.elapsed_time(b) * 1000 for a, b in timers)
    return {
        "workload": "B=1, 4 qk / 8 v heads, dk=dv=128, conv-fused decode step from a zero conv "
                    "state, in place",
        "graph_us_per_step": round(graph_us, 3),
        "steps_per_s": round(1e6 / graph_us, 1),
        "eager_us_per_step": round(eager, 2),
    }


def host_cost(device, calls=2000):
    """Host time of one eager GDNBackend call (indexed, T=1, 16/48 heads) at B=1 and B=8:
    `calls` back-to-back calls timed with the host clock, no synchronisation between them."""
    import torch

    from lightdelta_amd.backend import GDNBackend
    from lightdelta_amd.config import BackendConfig
    from lightdelta_amd.workloads import decode_case

    backend = GDNBackend(BackendConfig(compute="cuda_fused", state_io="indexed"))
    result = {}
    for batch in (1, 8):
        case = decode_case(batch, 1, num_k_heads=16, num_v_heads=48, pool_slots=batch + 2,
                           seed=0, device=device)
        args = [case[k] for k in ORDER]
        for _ in range(50):
            backend(*args, 1e-6)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(calls):
            backend(*args, 1e-6)
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        result[f"B{batch}_us_per_call"] = round((t1 - t0) / calls * 1e6, 2)
    result["workload"] = ("host time per eager GDNBackend call (validation, argument packing, "
                          "launch), 16/48 heads, T=1")
    return result


def tp_shares(steps, device):
    """The step at one GPU's share of the layer under head (tensor) parallelism: TP = 2 (8 qk
    / 16 v heads) and TP = 4 (4 qk / 8 v heads) at B = 32 and B = 128 requests per GPU.  Each
    GPU of a TP group runs exactly this launch on its own heads and state shard, with nothing
    exchanged inside the op.  `hot`: the same slots every step (keep policy); `cold`: disjoint
    slot sets rotated through at least 1 GiB of pool (stream policy)."""
    import torch

    from lightdelta_amd import ops
    from lightdelta_amd.workloads import decode_case

    saved = ops.state_cache_policy()
    slots_at, pool_at = ORDER.index("slots"), ORDER.index("pool")
    result = {"workload": "one GPU's share of the B-request step under head parallelism: "
                          "TP=2 (8 qk / 16 v heads), TP=4 (4 qk / 8 v heads); frac on state "
                          "bytes (one read + one write per tile) against the 8 TB/s HBM peak; "
                          "hot = the same slots every step, Infinity-Cache resident (keep "
                          "policy); cold = disjoint slot sets rotated through >= 1 GiB "
                          "(stream policy), the HBM-bound figure"}
    try:
        for tp in (2, 4):
            h, hv = H // tp, HV // tp
            for batch in (32, 128):
                case = decode_case(batch, 1, num_k_heads=h, num_v_heads=hv, seed=3,
                                   device=device)
                args = [case[k] for k in ORDER]
                tile_bytes = DIM * DIM * 4
                step_bytes = batch * hv * tile_bytes * 2
                ops.set_state_cache_policy("keep")
                hot = _graph_us(lambda: torch.ops.lightdelta.decode(*args, 1e-6), steps)
                per_set = batch * hv * tile_bytes
                sets = max(16, -(-(1 << 30) // per_set))
                big = torch.empty(sets * batch + 1, hv, DIM, DIM, device=device).normal_(0.0, 0.02)
                perm = torch.randperm(sets * batch, device=device) + 1
                slot_sets = [perm[i * batch:(i + 1) * batch].to(torch.int32).view(batch, 1)
                             for i in range(sets)]
                cold_args = list(args)
                cold_args[pool_at] = big

                def cold_pass():
                    for slots in slot_sets:
                        cold_args[slots_at] = slots
                        torch.ops.lightdelta.decode(*cold_args, 1e-6)

                ops.set_state_cache_policy("stream")
                cold = _graph_us(cold_pass, max(1, steps // sets)) / sets
                result[f"tp{tp}_b{batch}"] = {
                    "qk_heads": h, "v_heads": hv, "tiles": batch * hv,
                    "hot_us": round(hot, 3),
                    "hot_frac": round(step_bytes / hot / 1e3 / HBM_PEAK_GBS, 4),
                    "cold_us": round(cold, 3),
                    "cold_TBps": round(step_bytes / cold / 1e6, 3),
                    "cold_frac": round(step_bytes / cold / 1e3 / HBM_PEAK_GBS, 4),
                    "cold_pool_GiB": round(big.numel() * 4 / 2**30, 2),
                }
                del big, case, args, cold_args
    finally:
        ops.set_state_cache_policy(saved)
    return result


def prefill(device):
    """Prefill of 32 prompts x 1024 tokens, of one 4096-token prompt and of 1024 prompts x 32
    tokens (16 qk / 32 v heads, states from pool slots), timed over a few eager launches
    each, under every algorithm (token-serial recurrence; 64- or 32-token chunks in the WY
    form on the matrix cores); `auto_selects` is the form the default picks."""
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
        auto = _lib.load().ld_gdn_prefill_auto_chunked(total, seqs, HV)
        entry = {"auto_selects": {0: "token_serial", 64: "chunked", 32: "chunked_32"}[auto]}
        try:
            for algorithm in ("token_serial", "chunked", "chunked_32"):
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
                if algorithm != "token_serial":
                    # matrix-core work of the WY form per (chunk, v-head), in 16x16x4 fp32
                    # products and 16x16x32 bf16 ones: for 64 tokens the scan's 3,584 and the
                    # prep's 640 (forward substitution) and 80 bf16 (the q.k and k.k tiles);
                    # for 32 tokens the scan's 1,792 (counted once, as fp32 products, where it
                    # runs them as three bf16 ones), the prep's 8 (T10) and 12 bf16
                    c, scan, subst, tiles = ((64, 3584, 640, 80) if algorithm == "chunked"
                                             else (32, 1792, 8, 12))
                    chunk_flop = (scan + subst) * 2048 + tiles * 16384
                    flop = seqs * -(-length // c) * HV * chunk_flop
                    entry[algorithm]["mfma_TFLOPs"] = round(flop / ms / 1e9, 1)
            # new prompts (the serving case): no state read, zeros to start from; the form
            # AUTO picks
            ops.set_prefill_algorithm("auto")
            case["has_initial"].zero_()
            run()
            torch.cuda.synchronize()
            start, end = events()
            start.record()
            for _ in range(reps):
                run()
            end.record()
            torch.cuda.synchronize()
            ms = start.elapsed_time(end) / reps
            entry["fresh_auto"] = {"ms": round(ms, 3), "tokens_per_s": round(total / ms * 1e3, 1)}
        finally:
            ops.set_prefill_algorithm(saved)
        result[label] = entry
        del case
    result["workload"] = ("prefill (state from the slot, recurrence over the prompt, gated "
                          "RMSNorm, final state to the slot), 16 qk / 32 v heads; fresh_auto: "
                          "new prompts (zero initial state, no state read) under AUTO")
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
        us = replay_median(graph, 10)[0] / launches * 1e6
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
    beforehand, are captured as one HIP graph, replayed 10 times, each timed end to end
    (median reported); the verify launches alone are also timed per launch (HIP events)."""
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
    seconds = replay_median(graph, 10)[0]
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


def mtp_verify_cold(device, passes=4):
    """The B=64, T=4 verify step cache-cold: 8 disjoint sets of 256 slots (home + 3 per
    sequence) rotated through a 2049-slot (4 GiB) pool, stream policy, `passes` rounds of the
    8 sets captured in one HIP graph; one read and 4 writes of every tile (the commit is not
    part of this figure)."""
    import torch

    from lightdelta_amd import ops
    from lightdelta_amd.workloads import decode_case

    batch, width = 64, 4
    case = decode_case(batch, width, num_k_heads=H, num_v_heads=HV, pool_slots=8, seed=5,
                       device=device)
    big = torch.empty(2049, HV, DIM, DIM, device=device).normal_(0.0, 0.02)
    perm = torch.randperm(2048, device=device)[: 8 * batch * width] + 1
    sets = [perm[i * batch * width:(i + 1) * batch * width].to(torch.int32).view(batch, width)
            for i in range(8)]
    args = [case[k] for k in ORDER]
    args[ORDER.index("pool")] = big

    def rounds():
        for slots in sets:
            args[ORDER.index("slots")] = slots
            torch.ops.lightdelta.decode(*args, 1e-6)

    saved = ops.state_cache_policy()
    ops.set_state_cache_policy("stream")
    try:
        us = _graph_us(rounds, passes) / 8
    finally:
        ops.set_state_cache_policy(saved)
    nbytes = batch * HV * 65536 * (1 + width)
    del big
    return {
        "workload": "MTP verify B=64, T=4, 16 qk / 32 v heads, 8 disjoint slot sets rotated "
                    "through a 4 GiB pool (cache-cold), stream policy",
        "us_per_step": round(us, 2),
        "tokens_per_s": round(batch * width * 1e6 / us, 1),
        "bytes_per_step": nbytes,
        "TBps": round(nbytes / us / 1e6, 3),
        "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
    }


def stack48(steps, device, conv=False):
    """48 GDN decode layers captured as one HIP graph, batch 128, 16 qk / 32 v heads, 1024
    slots per layer (96 GiB fp32 state), stream cache policy; the slot ids (shared by every
    layer) are reshuffled before every replay by a device-to-device copy from a table of
    random distinct ids.  `steps` replays are timed end to end, reshuffles included.

    conv=True runs the serving layer's step instead: each layer is one decode_conv launch
    (the width-4 causal conv1d + SiLU on the pre-conv activations, fused in front of the
    GDN step) over its own 1024-slot bf16 conv pool of 3 columns (48 MiB per layer), the
    conv slot being the request's SSM slot."""
    import torch

    from lightdelta_amd import ops
    from lightdelta_amd.workloads import stack_case, stack_layer

    layers_n, batch, slots_n = 48, 128, 1024
    conv_len = 3 if conv else 0
    case = stack_case(layers_n, batch, pool_slots=slots_n, seed=5, device=device,
                      conv_len=conv_len)
    layers = [stack_layer(case, layer) for layer in range(layers_n)]

    if conv:
        def step():
            for a in layers:
                torch.ops.lightdelta.decode_conv(a["qkv"], a["conv_state"], a["conv_weight"],
                                                 None, *[a[k] for k in ORDER[1:]], 1e-6)
    else:
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
    ssm_bytes = layers_n * batch * HV * DIM * DIM * 4 * 2
    conv_bytes = layers_n * batch * case["qkv"].shape[-1] * conv_len * 2 * 2
    step_bytes = ssm_bytes + conv_bytes
    rate = steps / elapsed
    del case, layers, graph
    torch.cuda.empty_cache()
    what = ("conv-fused decode steps (decode_conv: causal conv1d + SiLU in front of the GDN "
            "step, a 3-column bf16 conv pool of 1024 slots per layer)" if conv else
            "decode steps")
    result = {
        "workload": f"48-layer stack of {what} in one HIP graph, batch 128, 16 qk / 32 v "
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
    if conv:
        result["conv_state_bytes_per_step"] = conv_bytes
    return result


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
        samples = [elapsed]
    else:
        graph = capture(step, args.steps)
        graph.replay()  # upload + warm the graph (untimed)
        torch.cuda.synchronize()
        # each sample times exactly K steps; the median sample is the figure
        elapsed, samples = replay_median(graph, args.samples)
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
        "timing": {"method": ("eager launches, one timed run" if args.no_graph else
                              f"one {args.steps}-step HIP graph replayed {len(samples)} times, "
                              "each replay timed with HIP events between synchronisations; "
                              "value = K / the median replay"),
                   "us_per_step": spread_us(samples, args.steps)},
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
            "regime": "Infinity-Cache resident: the workload steps the same 32 slots (64 MiB) in "
                      "place, which stay in the 256 MB Infinity Cache between steps; the "
                      "HBM-bound figures are `cold` and `stack48`",
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
        cold_elapsed, cold_samples = replay_median(cold_graph, args.samples)
        cold_steps = 16 * max(1, args.steps // 16)
        cold_rate = cold_steps / cold_elapsed
        result["cold"] = {
            "workload": "same step, 16 disjoint slot sets rotated through a 1024-slot (2 GiB) "
                        "pool; working set exceeds the 256 MB Infinity Cache",
            "cache_policy": "stream",
            "steps_per_s": round(cold_rate, 1),
            "us_per_step": spread_us(cold_samples, cold_steps),
            "state_TBps": round(STATE_BYTES * cold_rate / 1e12, 3),
            "frac": round(STATE_BYTES * cold_rate / 1e9 / HBM_PEAK_GBS, 4),
        }
        # the HBM-bound figure of the same kernel family, beside the cache-resident headline
        result["roofline"]["cold_frac"] = result["cold"]["frac"]
        result["roofline"]["cold_us_per_step"] = round(1e6 / cold_rate, 3)
        del big

    if not args.no_tp:
        result["tp_shares"] = tp_shares(args.steps, device)

    if not args.no_conv:
        result["conv_fused"] = conv_fused(case, op_args, args.steps, device)
        result["config1"] = config1(device, args.steps)

    if not args.no_table:
        result["operator_table"] = operator_table(device)
        result["host_cost"] = host_cost(device)

    if not args.no_prefill:
        result["prefill"] = prefill(device)

    if not args.no_mtp:
        result["mtp_verify"] = mtp_verify(args.steps, device)
        result["mtp_verify_cold"] = mtp_verify_cold(device)

    if not args.no_copies:
        result["copies"] = copies(device)

    if not args.no_stack:
        case = op_args = graph = None  # noqa: F841  (release the B=32 pools first)
        torch.cuda.empty_cache()
        if not args.no_stack_plain:
            result["stack48"] = stack48(args.stack_steps, device)
        if not args.no_conv:
            result["stack48_conv"] = stack48(args.stack_steps, device, conv=True)

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
