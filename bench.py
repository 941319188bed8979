"""Benchmark the complete LSSO mixer forward on one MI355X.

Workload (metric "mixer fwd tokens/s @B64 D256 H8 r32 L4096 fp16"):
LSSO(LSSOConfig(256, 8, 32, bias=True)) with seeded random compact-core
parameters, x ~ N(0, 1) FP16 [64, 4096, 256], shared default positions, no
mask.  One step is one forward x -> y including both
projections (reference protocol: benchmarks/benchmark_ball.py:156-208).

Prints one JSON line with the driver's fields plus
  roofline      the projection + reduction stage (at the headline shape the
                fused input projection + reduce kernel, the longest of the
                call) from HIP events that the library records around that
                stage in every timed step;
  settle        the untimed back-to-back steps run before the warmup so that
                the timed steps see the device's sustained clocks, with the
                per-step time of the same number of steps started cold;
  cpu_baseline  the CPU oracle (FP32 restatement of the reference CPU path)
                timed on this host on a bounded sample of the same workload.
On request (flags below) it also carries copy_ceiling (HBM copy, read and
write probes), clock_trace (shader clock after an idle gap) and
gemm_yardstick (the input projection alone as a plain GEMM, in hipBLASLt and
in this library).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

HBM_PEAK_GBPS = 8000.0
# Reference native CUDA forward at this exact shell: 10.135 ms per batch of
# 64 x 4096 tokens on one RTX 5070 Ti (results/cuda/wall_clock.csv:4).
REFERENCE_TOKENS_PER_S = 64 * 4096 / 10.135e-3


def parse_args() -> argparse.Namespace:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    # Defaults mirror the reference protocol's 50 warmup and 7 x 100 timed
    # iterations (benchmarks/benchmark_ball.py:156-208).  Runs of 100 steps
    # measured 3-4% slower per step than runs of 700-1000 on the same box.
    parser.add_argument("--steps", type=int, default=700)
    parser.add_argument("--warmup", type=int, default=50)
    parser.add_argument("--batch", type=int, default=None,
                        help="batch (default 64; 32 for --config c4)")
    parser.add_argument("--config", choices=("c3", "c4"), default="c3",
                        help="forward workload: c3 is the headline shell B64 D256 H8 r32 FP16 "
                             "(--length 1024 is config C2, 2048 and 4096 config C3); c4 is "
                             "B32 D384 H6 r64 BF16 with trailing-padding masks and per-sample "
                             "positions (config C4)")
    parser.add_argument("--length", type=int, default=None,
                        help="sequence length (default 4096; 2048 for --workload train)")
    parser.add_argument("--workload", choices=("forward", "train"), default="forward",
                        help="forward: the headline mixer forward (r=32); train: forward + "
                             "first-order backward of loss = mean(y^2) at r=48 (config C5)")
    parser.add_argument("--rank", type=int, default=None, choices=(16, 32, 48, 64),
                        help="--workload train only: rank (default 48, config C5; 32 is the "
                             "shell of the reference's published fwd+bwd numbers)")
    parser.add_argument("--cpu-samples", type=int, default=64,
                        help="sequences of the workload timed on the CPU oracle (0 skips)")
    parser.add_argument("--cpu-repeats", type=int, default=7)
    parser.add_argument("--no-parity", action="store_true",
                        help="skip the error figures against the CPU oracle")
    parser.add_argument("--slices", type=int, default=1,
                        help="forward only: split the batch into this many equal slices, one "
                             "layer call each, issued alternately on two streams of default "
                             "priority, so that one slice's compact solve can overlap another "
                             "slice's streaming kernels (A/B of that overlap; default 1 = one call)")
    parser.add_argument("--settle-ms", type=float, default=250.0,
                        help="before the warmup, run steps back to back for about this many "
                             "milliseconds of GPU time so that the timed steps see the device's "
                             "sustained clocks (0 disables; the JSON line reports the settle and the "
                             "per-step time of --steps steps started right after an idle gap)")
    parser.add_argument("--clock-trace", type=int, default=0,
                        help="forward only: after the timed region, idle, then run this many steps, "
                             "each followed by a one-wave shader-clock probe, and report the "
                             "projection + reduce kernel time and the clock over windows of steps")
    parser.add_argument("--copy-mib", type=int, default=0,
                        help="after the timed region, run one torch device copy of this many MiB "
                             "(reference kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE), then "
                             "the copy/read/write probes, and report their rates as copy_ceiling")
    parser.add_argument("--gemm-yardstick", type=int, default=0,
                        help="forward only: after the timed region, time this many calls each of the "
                             "input projection alone as a plain GEMM at the layer's shape (tokens x D "
                             "-> H (r + d)): torch's BF16 mm and linear (hipBLASLt) and this "
                             "library's linear_kernel, and report them as gemm_yardstick")
    return parser.parse_args()


STAGE_PROBE_STEPS = 10
TIMED_EVENT_EVERY = 4
# Idle time before the cold window of the settle phase: any idle gap of a few
# milliseconds restarts the device's clock transient.
SETTLE_IDLE_S = 0.05


def settle(run_step, settle_ms: float, cold_steps: int) -> dict | None:
    """Bring the device to its sustained clocks before a measurement.

    After an idle gap of a few milliseconds an MI355X runs about the first
    1.5 ms of work at full speed, then every kernel of the layer (the
    latency-bound solve as much as the streaming kernels) slows by up to a
    quarter for some tens of milliseconds before the clocks settle; a 20-step
    run that starts after a gap measures that dip, not the sustained rate.
    This function idles SETTLE_IDLE_S seconds, times `cold_steps` steps with
    events (the per-step time such a run measures), then runs steps back to
    back, with no host synchronization, for about `settle_ms` milliseconds of
    GPU time.  The caller continues without synchronizing until the
    synchronization that opens its timed region.  Returns the settle's record
    for the JSON line, or None when settle_ms is 0."""

    if settle_ms <= 0:
        return None
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    time.sleep(SETTLE_IDLE_S)
    begin.record()
    for _ in range(cold_steps):
        run_step()
    end.record()
    torch.cuda.synchronize()
    cold_ms = begin.elapsed_time(end) / cold_steps
    steps = max(1, int(settle_ms / cold_ms + 0.5))
    for _ in range(steps):
        run_step()
    return {
        "ms": settle_ms,
        "steps": steps,
        "cold_steps": cold_steps,
        "cold_ms_per_step": cold_ms,
        "note": (f"untimed steps run back to back before the warmup; cold_ms_per_step is the event "
                 f"time per step of {cold_steps} steps started after {SETTLE_IDLE_S * 1e3:.0f} ms idle"),
    }


def copy_ceiling(mib, device):
    """Device-copy rates on buffers of `mib` MiB, after the timed region.

    First one torch `copy_` (ROCm's `__amd_rocclr_copyBuffer`), the dispatch
    that scales rocprofv3's FETCH_SIZE / WRITE_SIZE; then the probes of
    liblsso_probe_gfx950.so (one 16-byte vector per thread: a plain copy, the
    same with the nontemporal hint, a read, a write, and the write as a raw
    buffer store under cache-policy operands 0, 2 (nt), 16 (sc1) and 18),
    five launches each
    on torch's current stream, timed with events around each launch.
    Returns {probe: {"bytes", "ms", "GB/s"}} with the median time.
    """
    import ctypes
    from lsso_amd.build import probe_library_path

    source = torch.empty(mib << 20, dtype=torch.uint8, device=device).fill_(1)
    target = torch.empty_like(source)
    sink = torch.zeros(4, dtype=torch.int32, device=device)
    torch.cuda.synchronize()
    rates = {}
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    target.copy_(source)
    stop.record()
    torch.cuda.synchronize()
    nbytes = source.numel()
    rates["torch_copy"] = {"bytes": 2 * nbytes, "ms": start.elapsed_time(stop)}
    path = probe_library_path()
    if path.exists():
        probe = ctypes.CDLL(str(path))
        probe.lsso_probe_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
                                          ctypes.c_int, ctypes.c_void_p]
        probe.lsso_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
                                          ctypes.c_void_p]
        probe.lsso_probe_write.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p]
        probe.lsso_probe_write_policy.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int,
                                                  ctypes.c_void_p]
        stream = torch.cuda.current_stream(device).cuda_stream
        src, dst = source.data_ptr(), target.data_ptr()
        probes = {
            "probe_copy": (2 * nbytes, lambda: probe.lsso_probe_copy(src, dst, nbytes, 0, stream)),
            "probe_copy_streaming": (2 * nbytes,
                                     lambda: probe.lsso_probe_copy(src, dst, nbytes, 1, stream)),
            "probe_read": (nbytes, lambda: probe.lsso_probe_read(src, sink.data_ptr(), nbytes, stream)),
            "probe_write": (nbytes, lambda: probe.lsso_probe_write(dst, nbytes, stream)),
            **{f"probe_write_policy_{policy}": (
                nbytes, lambda policy=policy: probe.lsso_probe_write_policy(dst, nbytes, policy, stream))
               for policy in (0, 2, 16, 18)},
        }
        for name, (moved, launch) in probes.items():
            pairs = []
            for _ in range(5):
                begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                begin.record()
                code = launch()
                end.record()
                if code != 0:
                    raise RuntimeError(f"{name} failed with code {code}")
                pairs.append((begin, end))
            torch.cuda.synchronize()
            rates[name] = {"bytes": moved, "ms": statistics.median(b.elapsed_time(e) for b, e in pairs)}
    for entry in rates.values():
        entry["GB/s"] = entry["bytes"] / (entry["ms"] * 1e-3) / 1e9
    del source, target, sink
    return rates
def gemm_yardstick(x, weight, bias, calls: int) -> dict:
    """The input projection alone as a plain GEMM at the layer's shape.

    x [B, L, D] (FP16 or BF16), weight [W, D] and bias [W] (FP32): torch's
    BF16 `mm` and `linear` (hipBLASLt kernels on ROCm) on BF16 copies of the
    operands, and this library's `linear_kernel` (x as given, BF16 output,
    FP32 bias, the unfused input projection of the layer).  Each case runs
    `calls` untimed calls, then `calls` calls with events around each one on
    torch's current stream.  Returns {case: {"median_us", "mean_us", "GB/s",
    "TFLOP/s"}} with bytes = x read + output written (2 bytes each) and
    flops = 2 M N K.
    """
    from lsso_amd.ball import hip

    rows, depth = x.shape[0] * x.shape[1], x.shape[2]
    width = weight.shape[0]
    x_bf16 = x.reshape(rows, depth).bfloat16()
    w_bf16 = weight.bfloat16()
    w_t = w_bf16.t().contiguous()
    b_bf16 = bias.bfloat16()
    cases = {
        "torch_mm_bf16": lambda: torch.mm(x_bf16, w_t),
        "torch_linear_bf16": lambda: torch.nn.functional.linear(x_bf16, w_bf16, b_bf16),
        "lsso_linear_kernel": lambda: hip.linear(x, weight, bias, torch.bfloat16),
    }
    moved = rows * depth * 2 + rows * width * 2
    flops = 2 * rows * width * depth
    out = {}
    with torch.inference_mode():
        for name, call in cases.items():
            for _ in range(calls):
                call()
            events = [torch.cuda.Event(enable_timing=True) for _ in range(2 * calls)]
            for i in range(calls):
                events[2 * i].record()
                call()
                events[2 * i + 1].record()
            torch.cuda.synchronize()
            times = [events[2 * i].elapsed_time(events[2 * i + 1]) * 1e3 for i in range(calls)]
            median = statistics.median(times)
            out[name] = {"median_us": median, "mean_us": statistics.mean(times),
                         "GB/s": moved / (median * 1e-6) / 1e9, "TFLOP/s": flops / (median * 1e-6) / 1e12}
    del x_bf16, w_bf16, w_t, b_bf16
    return out


CLOCK_SPINS = 300  # about 5 us of one dependent FMA chain per clock probe
CLOCK_WINDOWS = (0, 5, 10, 20, 50, 100, 200, 400, 1000)


def clock_trace(run_step, make_events, slot: int, steps: int, device) -> dict:
    """Kernel time and shader clock per step from a cold start.

    After SETTLE_IDLE_S seconds idle, `steps` steps run back to back, each
    followed by lsso_probe_clock (one wave, CLOCK_SPINS dependent FMAs between
    two reads of the shader-clock and constant-rate counters).  Events bracket
    stage `slot` of each step.  Returns the mean kernel time and clock over
    the windows of steps in CLOCK_WINDOWS."""

    import ctypes
    from lsso_amd.build import probe_library_path

    probe = ctypes.CDLL(str(probe_library_path()))
    probe.lsso_probe_clock.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    rate_khz = probe.lsso_probe_wall_clock_khz()
    if rate_khz <= 0:
        raise RuntimeError(f"lsso_probe_wall_clock_khz failed with code {rate_khz}")
    records = torch.zeros(steps, 4, dtype=torch.int64, device=device)
    step_events = []
    for _ in range(steps):
        events = [None] * 8
        events[2 * slot], events[2 * slot + 1] = make_events(2)
        step_events.append(events)
    stream = torch.cuda.current_stream(device).cuda_stream
    torch.cuda.synchronize()
    time.sleep(SETTLE_IDLE_S)
    for index in range(steps):
        run_step(step_events[index])
        code = probe.lsso_probe_clock(records[index].data_ptr(), CLOCK_SPINS, stream)
        if code != 0:
            raise RuntimeError(f"lsso_probe_clock failed with code {code}")
    torch.cuda.synchronize()
    counts = records.cpu().tolist()
    kernel_us = [ev[2 * slot].elapsed_time(ev[2 * slot + 1]) * 1e3 for ev in step_events]
    clock_ghz = [c[0] / c[1] * rate_khz / 1e6 for c in counts]
    windows = []
    edges = [edge for edge in CLOCK_WINDOWS if edge < steps] + [steps]
    for low, high in zip(edges[:-1], edges[1:]):
        windows.append({"steps": [low, high],
                        "kernel_us": statistics.mean(kernel_us[low:high]),
                        "clock_ghz": statistics.mean(clock_ghz[low:high])})
    return {"steps": steps, "idle_ms": SETTLE_IDLE_S * 1e3, "probe_spins": CLOCK_SPINS, "windows": windows}


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "mixer_forward_c3_l4096_hbm_traffic.md")


def measured_traffic(kernel_prefix: str):
    """(kernel name, HBM bytes per launch) of the first kernel whose name
    starts with `kernel_prefix` in the calibrated rocprofv3
    FETCH_SIZE/WRITE_SIZE summary committed under profiles/ for the headline
    workload, or (None, None) when the summary has no such line."""

    try:
        with open(TRAFFIC_FILE) as handle:
            for line in handle:
                if line.startswith("traffic_bytes_per_launch:"):
                    name, _, value = line.split(":", 1)[1].rpartition("=")
                    if name.strip().startswith(kernel_prefix):
                        return name.strip(), float(value)
    except OSError:
        return None, None
    return None, None


def error_figures(actual: torch.Tensor, expected: torch.Tensor) -> dict:
    """max_abs = max |a - e|, max_rel = max |a - e| / max |e|, rel_l2 =
    ||a - e|| / ||e||, in FP64."""

    a = actual.detach().to(device="cpu", dtype=torch.float64)
    e = expected.detach().to(device="cpu", dtype=torch.float64)
    diff = (a - e).abs()
    return {
        "max_abs": float(diff.max()),
        "max_rel": float(diff.max() / e.abs().max()),
        "rel_l2": float((a - e).norm() / e.norm()),
    }


def cpu_baseline(layer, x_cpu: torch.Tensor, samples: int, repeats: int, mask=None,
                 position_ids=None) -> tuple[dict, torch.Tensor]:
    """Time the CPU oracle (reference CPU path restated, FP32) on `samples`
    sequences of the workload; tokens/s is scaled by the sample size.
    Returns the record and the oracle's FP32 output for those sequences."""

    from oracle import lsso_reference as oracle

    cores = min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "1024")))
    torch.set_num_threads(cores)
    params = {name: p.detach().float().cpu() for name, p in layer.named_parameters()}
    config = {"dim": layer.config.dim, "num_heads": layer.config.num_heads,
              "rank": layer.config.rank, "bias": layer.config.bias}
    x = x_cpu[:samples].contiguous()
    sample_mask = None if mask is None else mask[:samples]
    sample_positions = None if position_ids is None else position_ids[:samples]
    with torch.no_grad():
        output = oracle.lsso_forward(params, config, x, sample_mask, sample_positions)  # warmup
        times = []
        for _ in range(repeats):
            start = time.perf_counter()
            oracle.lsso_forward(params, config, x, sample_mask, sample_positions)
            times.append(time.perf_counter() - start)
    seconds = statistics.median(times)
    tokens = x.shape[0] * x.shape[1]
    model = ""
    try:
        with open("/proc/cpuinfo") as handle:
            for line in handle:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": tokens / seconds,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{x.shape[0]} of {x_cpu.shape[0]} sequences x {x.shape[1]} tokens, FP32 CPU oracle "
                  f"(oracle/lsso_reference.py), median of {repeats} after 1 warmup, "
                  f"{seconds * 1e3:.1f} ms per sample batch",
        "cpu": model,
    }, output


def parity(layer, x_cpu: torch.Tensor, y: torch.Tensor, fp32_output: torch.Tensor | None,
           fp32_samples: int, mask=None, position_ids=None) -> dict:
    """Error figures of the GPU output y against the FP32 CPU oracle (on the
    sequences the CPU baseline ran, or on 3 when it did not run) and its
    rel-L2 error against the FP64 oracle on sequences 0, B/2 and B-1."""

    from oracle import lsso_reference as oracle

    config = {"dim": layer.config.dim, "num_heads": layer.config.num_heads,
              "rank": layer.config.rank, "bias": layer.config.bias}
    if fp32_output is None:
        fp32_samples = min(3, x_cpu.shape[0])
        params = {name: p.detach().float().cpu() for name, p in layer.named_parameters()}
        with torch.no_grad():
            fp32_output = oracle.lsso_forward(
                params, config, x_cpu[:fp32_samples].contiguous(),
                None if mask is None else mask[:fp32_samples],
                None if position_ids is None else position_ids[:fp32_samples])
    figures = error_figures(y[:fp32_samples], fp32_output)
    picks = sorted({0, x_cpu.shape[0] // 2, x_cpu.shape[0] - 1})
    params64 = {name: p.detach().double().cpu() for name, p in layer.named_parameters()}
    with torch.no_grad():
        fp64_output = oracle.lsso_forward(params64, config, x_cpu[picks].double(),
                                          None if mask is None else mask[picks],
                                          None if position_ids is None else position_ids[picks])
    figures["rel_l2_fp64"] = error_figures(y[picks], fp64_output)["rel_l2"]
    figures["reference"] = (f"FP32 CPU oracle on sequences 0..{fp32_samples - 1} (max_rel = max|a-e| / "
                            f"max|e|); FP64 oracle on sequences {picks}")
    figures["limit_rel_l2_fp64"] = 5e-3
    return figures


def train_benchmark(args: argparse.Namespace) -> int:
    """Forward + analytic backward of the complete mixer (config C5: B=64,
    D=256, H=8, r=48, L=2048, FP16 x, loss = mean(y^2), gradients for x and
    all seven parameters); tokens/s of whole training steps.  --rank 32 runs
    the shell of the reference's published fwd+bwd numbers and reports the
    ratio to them as vs_baseline."""

    from lsso_amd import LSSO, LSSOConfig

    device = torch.device("cuda", 0)
    length = 2048 if args.length is None else args.length
    rank = 48 if args.rank is None else args.rank
    batch, dim, heads = args.batch, 256, 8
    torch.manual_seed(0)
    layer = LSSO(LSSOConfig(dim=dim, num_heads=heads, rank=rank, bias=True))
    with torch.no_grad():
        layer.core_base_raw.normal_(std=0.05)
        layer.core_drive_weight.normal_(std=0.05)
    layer = layer.to(device).train()
    x = torch.randn(batch, length, dim, generator=torch.Generator().manual_seed(1)).half().to(device)
    x.requires_grad_(True)

    def step() -> None:
        x.grad = None
        for parameter in layer.parameters():
            parameter.grad = None
        y = layer(x, implementation="hip")
        y.float().square().mean().backward()

    settled = settle(step, args.settle_ms, args.steps)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    grads = [x.grad] + [parameter.grad for parameter in layer.parameters()]
    if any(g is None or not torch.isfinite(g).all() for g in grads):
        print("a gradient of the last timed step is missing or not finite", file=sys.stderr)
        return 1
    tokens = batch * length
    # The reference publishes fwd+bwd only for the r = 32 shell at B = 64
    # (RTX 5070 Ti, results/cuda/wall_clock.csv:5-7): B*L / (7.512, 15.260,
    # 29.160 ms) at L = 1024, 2048, 4096.
    published = {1024: 64 * 1024 / 7.512e-3, 2048: 64 * 2048 / 15.260e-3, 4096: 64 * 4096 / 29.160e-3}
    value = tokens * args.steps / elapsed
    vs_baseline = value / published[length] if rank == 32 and batch == 64 and length in published else None
    result = {
        "metric": f"mixer fwd+bwd tokens/s @B{batch} D256 H8 r{rank} L{length} fp16",
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": 1e3 * elapsed / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": vs_baseline,
        "dtype": "bf16",
        "data": "synthetic: x ~ N(0,1) fp16, seeded random-init weights",
        "config": {"workload": "lsso_mixer_forward_backward", "batch": batch, "length": length,
                   "dim": dim, "heads": heads, "rank": rank, "bias": True, "io_dtype": "fp16",
                   "grad_dtype": "fp32 parameters, fp16 x", "loss": "mean(y^2)"},
    }
    if settled is not None:
        result["settle"] = settled
    print(json.dumps(result), flush=True)
    return 0


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
            "(every GPU box in this build has one MI355X).",
            file=sys.stderr,
        )
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm device", file=sys.stderr)
        return 2

    from lsso_amd import LSSO, LSSOConfig
    from lsso_amd.ball import hip

    hip.load()
    if args.workload == "train":
        if args.batch is None:
            args.batch = 64
        return train_benchmark(args)
    device = torch.device("cuda", 0)
    if args.length is None:
        args.length = 4096
    masked = args.config == "c4"
    if args.batch is None:
        args.batch = 32 if masked else 64
    if masked:
        batch, length, dim, heads, rank = args.batch, args.length, 384, 6, 64
    else:
        batch, length, dim, heads, rank = args.batch, args.length, 256, 8, 32
    torch.manual_seed(0)
    layer = LSSO(LSSOConfig(dim=dim, num_heads=heads, rank=rank, bias=True))
    with torch.no_grad():
        layer.core_base_raw.normal_(std=0.05)
        layer.core_drive_weight.normal_(std=0.05)
    layer = layer.to(device).eval()
    generator = torch.Generator().manual_seed(1)
    mask_cpu = position_ids_cpu = None
    if masked:
        # C4: valid lengths ~ U[L/4, L] with trailing padding, per-sample
        # positions start_b + arange(L) with start_b ~ U[0, 1024).
        lengths = torch.randint(length // 4, length + 1, (batch,), generator=generator)
        mask_cpu = torch.arange(length)[None, :] < lengths[:, None]
        starts = torch.randint(0, 1024, (batch,), generator=generator)
        position_ids_cpu = starts[:, None] + torch.arange(length)[None, :]
        x_cpu = torch.randn(batch, length, dim, generator=generator).bfloat16()
    else:
        x_cpu = torch.randn(batch, length, dim, generator=generator).half()
    x = x_cpu.to(device)
    mask = None if mask_cpu is None else mask_cpu.to(device)
    position_ids = None if position_ids_cpu is None else position_ids_cpu.to(device)
    tokens = batch * length

    w_bc, b_bc = layer.w_bc.weight, layer.w_bc.bias
    w_o, b_o = layer.w_o.weight, layer.w_o.bias
    base, drive, eta_raw = layer.core_base_raw, layer.core_drive_weight, layer.eta_raw

    # The step is exactly the module's native inference forward for an
    # unmasked input with default positions (lsso_amd/ball/model.py,
    # _forward_native): one lsso_hip_layer_forward call (input projection
    # fused with the token reductions, compact solve, apply fused with the
    # output projection).  The library records HIP events around its stages
    # on the launch stream (lsso_hip_layer_forward_timed).
    stage_names = ("phase_table", "project_reduce", "solve", "mix_project")
    width = heads * rank + dim
    io_bytes = 2  # FP16 or BF16 x and y
    with torch.inference_mode():
        centered_positions, valid_counts, row_mask = layer._native_geometry(x, mask, position_ids)
    # Which kernels the layer call runs: the input projection is fused with
    # the reductions up to rank 32 (LSSO_HIP_FUSED_PROJECTION=1 or 0 makes the
    # library fuse at every rank or never), and the apply with the output
    # projection inside the fused readout's envelope
    # (lsso_hip_mixer_projected_supported).
    fused_in = {"1": True, "0": False}.get(os.environ.get("LSSO_HIP_FUSED_PROJECTION", ""), rank <= 32)
    probe = torch.empty(1, 1, width, dtype=torch.bfloat16, device=device)
    fused_out = hip.mix_project_supported(probe, layer.core_base_raw, layer.core_drive_weight,
                                          layer.eta_raw)
    del probe
    # Algorithmic bytes per launch, counting the ABI tensors once (the FP32
    # partials and apply records in the workspace are left out):
    #   project_reduce: x read (FP16) + packed write (BF16) + W_in, b_in (FP32)
    #   mix_project:    packed read (BF16) + y write (FP16) + W_o, b_o (FP32)
    # Outside the fused envelopes a stage runs two kernels with a BF16
    # round trip between them (packed written and read back, or mixed), and
    # its bytes count both.
    stage_kernels = {
        "project_reduce": (
            "lsso_hip::project_reduce_kernel<",
            tokens * (dim * io_bytes + width * 2) + width * dim * 4 + width * 4,
            "fused input projection + token reductions (x -> packed, G, S)",
        ) if fused_in else (
            "lsso_hip::linear_kernel<",
            tokens * (dim * io_bytes + 2 * width * 2) + width * dim * 4 + width * 4,
            "input projection then token reductions (x -> packed -> G, S)",
        ),
        "mix_project": (
            "lsso_hip::mix_project_kernel<",
            tokens * (width * 2 + dim * io_bytes) + dim * dim * 4 + dim * 4,
            "fused apply + output projection (packed -> y)",
        ) if fused_out else (
            "lsso_hip::apply_kernel<",
            tokens * (width * 2 + 2 * dim * 2 + dim * io_bytes) + dim * dim * 4 + dim * 4,
            "apply then output projection (packed -> mixed -> y)",
        ),
    }

    def step(events) -> torch.Tensor:
        return hip.layer_forward(x, w_bc, b_bc, base, drive, eta_raw, centered_positions, valid_counts,
                                 w_o, b_o, row_mask=row_mask, stage_events=events)

    slices = args.slices
    if slices < 1 or batch % slices:
        print(f"--slices {slices} must divide the batch {batch}", file=sys.stderr)
        return 2
    if slices > 1 and masked:
        print("--slices is only wired for the unmasked workload", file=sys.stderr)
        return 2
    launch_stream = torch.cuda.current_stream(device)
    slice_streams = [torch.cuda.Stream(device) for _ in range(2)] if slices > 1 else []
    per_slice = batch // slices

    def sliced_step(events) -> list:
        # Slice k runs on stream k % 2; the events (if any) go with slice 0.
        outputs = []
        for stream in slice_streams:
            stream.wait_stream(launch_stream)
        for k in range(slices):
            with torch.cuda.stream(slice_streams[k % 2]):
                rows = slice(k * per_slice, (k + 1) * per_slice)
                outputs.append(hip.layer_forward(x[rows], w_bc, b_bc, base, drive, eta_raw, centered_positions,
                                                 valid_counts, w_o, b_o, row_mask=None,
                                                 stage_events=events if k == 0 else None))
        for stream in slice_streams:
            launch_stream.wait_stream(stream)
        return outputs

    def timed_step(events) -> None:
        if slices == 1:
            step(events)
        else:
            sliced_step(events)

    def recorded_events(count):
        # torch creates the HIP event on its first record.
        events = [torch.cuda.Event(enable_timing=True) for _ in range(count)]
        for event in events:
            event.record()
        return events

    with torch.inference_mode():
        reference_out = layer(x, valid_mask=mask, position_ids=position_ids, implementation="hip")
        check = step(None)
        projected = hip.linear(x, w_bc, b_bc, torch.bfloat16, row_mask=row_mask)
        mixed = hip.forward_inference(projected, base, drive, eta_raw, centered_positions, valid_counts)
        three_calls = hip.linear(mixed, w_o, b_o, x.dtype, row_mask=row_mask)
        del projected, mixed
        if not (torch.equal(check, reference_out) and torch.equal(check, three_calls)):
            print("the layer step differs from LSSO.forward(implementation='hip') or from "
                  "linear -> forward_inference -> linear", file=sys.stderr)
            return 1
        del three_calls
        if slices > 1:
            # Results do not depend on the batch composition, so the slices
            # reproduce the one-call output bit for bit.
            if not torch.equal(torch.cat(sliced_step(None), 0), check):
                print(f"the {slices}-slice step differs from the one-call step", file=sys.stderr)
                return 1
        # Per-stage times from untimed steps with events on all four stages
        # (the library's kernel dispatches record them).  Events on every
        # stage still add about ten microseconds to a step, so the timed
        # steps carry only the two of the projection + reduction stage, the
        # longest stage of every workload here, and only every
        # TIMED_EVENT_EVERY-th timed step carries them (a pair on every step
        # measured 0.2283 against 0.2255 ms per step without).  Every event
        # exists before the settle, so nothing between the settle and the
        # timed region waits on the host.
        stage_events = [recorded_events(8) for _ in range(STAGE_PROBE_STEPS)]
        slot = stage_names.index("project_reduce")
        timed_events = [[None] * 8 for _ in range(args.steps)]
        timed_pairs = []
        for index in range(0, args.steps, TIMED_EVENT_EVERY):
            pair = recorded_events(2)
            timed_events[index][2 * slot], timed_events[index][2 * slot + 1] = pair
            timed_pairs.append(pair)
        settled = settle(lambda: timed_step(None), args.settle_ms, args.steps)
        for events in stage_events:
            step(events)
        for _ in range(args.warmup):
            timed_step(None)
        torch.cuda.synchronize()
        start = time.perf_counter()
        for index in range(args.steps):
            timed_step(timed_events[index])
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - start

    stage_ms = {
        name: statistics.mean(ev[2 * k].elapsed_time(ev[2 * k + 1]) for ev in stage_events)
        for k, name in enumerate(stage_names)
    }
    dominant = stage_names[slot]
    copy_rates = copy_ceiling(args.copy_mib, device) if args.copy_mib > 0 else None
    yardstick = gemm_yardstick(x, w_bc, b_bc, args.gemm_yardstick) if args.gemm_yardstick > 0 else None
    clocks = None
    if args.clock_trace > 0:
        with torch.inference_mode():
            clocks = clock_trace(step, recorded_events, slot, args.clock_trace, device)

    ms_per_step = 1e3 * elapsed / args.steps
    value = tokens * args.steps / elapsed
    kernel_ms = statistics.mean(start_event.elapsed_time(end_event) for start_event, end_event in timed_pairs)
    kernel_prefix, kernel_bytes, kernel_role = stage_kernels[dominant]
    if slices > 1:
        # The timed events bracket slice 0's launch of the dominant kernel,
        # which streams 1 / slices of the tokens and reads the weights once.
        weight_bytes = dim * dim * 4 + dim * 4 if dominant == "mix_project" else width * dim * 4 + width * 4
        kernel_bytes = (kernel_bytes - weight_bytes) // slices + weight_bytes
    achieved = kernel_bytes / (kernel_ms * 1e-3) / 1e9
    # HBM bytes per token the chain moves by design: x read, packed written
    # and read back (BF16), y written; plus a second packed read when the
    # input projection is not fused with the reductions and a mixed round
    # trip (BF16) when the apply is not fused with the output projection.
    chain_bytes_per_token = (dim * io_bytes + 2 * width * 2 + dim * io_bytes
                             + (0 if fused_in else width * 2) + (0 if fused_out else 2 * dim * 2))
    chain_bytes = tokens * chain_bytes_per_token
    headline = (batch, length) == (64, 4096) and not masked and slices == 1
    kernel_name, traffic = measured_traffic(kernel_prefix) if headline else (None, None)
    if kernel_name is None:
        kernel_name = kernel_prefix.rstrip("<")
    io_name = "bf16" if masked else "fp16"
    result = {
        "metric": ("mixer fwd tokens/s @B64 D256 H8 r32 L4096 fp16; % HBM roofline" if headline else
                   f"mixer fwd tokens/s @B{batch} D{dim} H{heads} r{rank} L{length} {io_name}"
                   + (" masked" if masked else "") + (f" in {slices} slices on 2 streams" if slices > 1 else "")),
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": value / REFERENCE_TOKENS_PER_S if headline else None,
        "dtype": "bf16",
        "data": (f"synthetic: x ~ N(0,1) {io_name}, seeded random-init weights"
                 + ("; valid lengths ~ U[L/4, L] with trailing padding, per-sample positions "
                    "start ~ U[0, 1024); tokens/s counts all B*L rows" if masked else "")),
        "config": {
            "workload": "lsso_mixer_forward",
            "batch": batch,
            "length": length,
            "dim": dim,
            "heads": heads,
            "rank": rank,
            "bias": True,
            "io_dtype": io_name,
            "packed_dtype": "bf16",
            "positions": "per-sample" if masked else "default",
            "mask": masked,
            "slices": slices,
            "fused_input_projection": fused_in,
            "fused_output_projection": fused_out,
            "accumulate_dtype": "fp32",
            "chain_bytes_per_token": chain_bytes_per_token,
            "chain_hbm_fraction": chain_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBPS,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"{kernel_name} ({kernel_role})",
            "achieved": achieved,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBPS,
            "traffic": traffic,
            "traffic_source": ("profiles/mixer_forward_c3_l4096_hbm_traffic.md (rocprofv3 FETCH_SIZE + "
                               "WRITE_SIZE, copy-calibrated)") if traffic is not None else None,
            "avg_ms": kernel_ms,
            "avg_ms_launches": f"{len(timed_pairs)} of the {args.steps} timed launches (every {TIMED_EVENT_EVERY}th step)",
            "stage_ms": stage_ms,
            "stage_ms_source": f"{STAGE_PROBE_STEPS} untimed steps with events around every stage",
        },
    }
    if settled is not None:
        result["settle"] = settled
    fp32_output = None
    samples = min(args.cpu_samples, batch)
    if args.cpu_samples > 0:
        result["cpu_baseline"], fp32_output = cpu_baseline(layer, x_cpu, samples, args.cpu_repeats,
                                                           mask_cpu, position_ids_cpu)
    if not args.no_parity:
        result["parity"] = parity(layer, x_cpu, check, fp32_output, samples, mask_cpu, position_ids_cpu)
    if copy_rates is not None:
        result["copy_ceiling"] = copy_rates
    if yardstick is not None:
        result["gemm_yardstick"] = yardstick
    if clocks is not None:
        clocks["kernel"] = kernel_name
        result["clock_trace"] = clocks
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
