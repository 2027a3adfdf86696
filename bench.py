"""Benchmark of the MI355X MSDA kernels on the BASELINE headline workload.

One step = one forward and one backward of ``deformops_amd.registry.msda`` on
config 4 (Mask2Former pixel-decoder encoder, large): B=4, levels 128x128, 64x64,
32x32 (Q = S = 21,504), H=8, D=32, P=4, bfloat16 value, weights and locations,
linear method, synthetic seeded inputs already resident in HBM.

Prints one JSON line: ``value`` is fwd+bwd milliseconds per call (lower is
better); ``roofline`` rates the dominant launch, the backward C-ABI call (its
kernels run back to back on one stream), by its algorithmic bytes over its average
duration, timed with HIP events on that stream; ``cpu_baseline`` times the torch
restatement of the reference's eager CPU path on a bounded sample of the same
workload, scaled to one full call.

    python bench.py [--steps K] [--warmup W] [--dtype bf16|f16|f32] [--loc-dtype ...]
                    [--method linear|softmax] [--config 0..4]

``--config`` measures another BASELINE configuration the same way (config 4, the
headline, is the default and the only one the driver's line is quoted on). The
``roofline.traffic`` figure is the profiled one of config 4 (bf16, linear) and is
null for every other workload.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import torch

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

from tests.workloads import CONFIGS, algorithmic_bytes, make_workload  # noqa: E402

METRIC = "MSDA fwd+bwd ms/call + achieved HBM GB/s, 21.5k-query bf16 encoder, 1 GPU"
PEAK_HBM_GBS = 8000.0
# HBM bytes of one backward C-ABI call on the default workload (bf16 value, weights
# and locations, linear method): rocprofv3 FETCH_SIZE x 2 + WRITE_SIZE x 1, summed
# over the call's kernels, each counter scaled by what it reads for a 256 MiB copy.
# profiles/msda_config4_bf16_hbm_traffic.md holds the passes and the calibration.
BACKWARD_TRAFFIC_BYTES = 1_129_519_424
DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _events(n: int) -> list[torch.cuda.Event]:
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def time_fwd_bwd(w, steps: int, warmup: int, softmax: bool):
    """Time K full fwd+bwd steps through the public API; per-step events + wall clock."""
    from deformops_amd.registry import msda  # noqa: PLC0415

    value, shapes, starts, loc, attn = w.operands(softmax=softmax)
    leaves = [t.detach().clone().requires_grad_(True) for t in (value, loc, attn)]
    method = "softmax" if softmax else "linear"

    def step() -> None:
        for leaf in leaves:
            leaf.grad = None
        out = msda(leaves[0], shapes, starts, leaves[1], leaves[2], method=method)
        out.backward(w.grad_output)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    starts_ev, ends_ev = _events(steps), _events(steps)
    t0 = time.perf_counter()
    for i in range(steps):
        starts_ev[i].record()
        step()
        ends_ev[i].record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    per_step = [s.elapsed_time(e) for s, e in zip(starts_ev, ends_ev)]
    return wall_ms / steps, statistics.median(per_step)


def time_kernels(w, steps: int, warmup: int, softmax: bool) -> dict[str, float]:
    """Average device time of each direction alone, through the C ABI, on torch's stream.

    The forward is one kernel. The backward call launches the bucket sort of the
    samples (clear, count, scan, place), the per-unit softmax statistics (softmax
    only), the owner-computes grad_value kernel (which also zeroes positions no level
    covers) and the location / weight gradient kernel, all on this stream; the events
    bracket the whole call.
    """
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    lib = _lib.load()
    value, shapes, starts, loc, attn = w.operands(softmax=softmax)
    B, S, H, D, Q, L, P = w.sizes
    out = torch.empty((B, Q, H * D), dtype=value.dtype, device=value.device)
    gv = torch.empty_like(value)
    gl = torch.empty_like(loc)
    ga = torch.empty_like(attn)
    stream = torch.cuda.current_stream()
    flags = _lib.FLAG_SOFTMAX if softmax else 0
    vcode, lcode = _lib.DTYPE_CODES[value.dtype], _lib.DTYPE_CODES[loc.dtype]
    icode = _lib.INDEX_CODES[shapes.dtype]

    def fwd() -> None:
        lib.check(lib.forward(value.data_ptr(), vcode, shapes.data_ptr(), starts.data_ptr(), icode,
                              loc.data_ptr(), lcode, attn.data_ptr(), out.data_ptr(),
                              B, S, H, D, Q, L, P, flags, stream.cuda_stream))

    def bwd() -> None:
        lib.check(lib.backward(value.data_ptr(), vcode, shapes.data_ptr(), starts.data_ptr(), icode,
                               loc.data_ptr(), lcode, attn.data_ptr(), w.grad_output.data_ptr(),
                               gv.data_ptr(), gl.data_ptr(), ga.data_ptr(),
                               B, S, H, D, Q, L, P, flags, stream.cuda_stream))

    result = {}
    for name, fn in (("forward", fwd), ("backward", bwd)):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        times = []
        for _ in range(steps):
            s, e = _events(2)
            s.record(stream)
            fn()
            e.record(stream)
            times.append((s, e))
        torch.cuda.synchronize()
        result[name] = statistics.mean(s.elapsed_time(e) for s, e in times)
    return result


def cpu_baseline(config: int, dtype: torch.dtype, loc_dtype: torch.dtype, softmax: bool) -> dict:
    """The reference's eager CPU path (torch restatement) on a bounded sample.

    Sample: batch 1 and at most the first 21,504 queries of the configuration (at
    config 4, one image: 21,504 of the 86,016 (batch, query) pairs), same dtype;
    1 warm-up and 3 timed fwd + autograd-bwd iterations, median, scaled by the
    call's (batch, query) pairs over the sample's.
    """
    from oracle.eager import eager_msda  # noqa: PLC0415

    cfg = CONFIGS[config]
    queries = make_workload(cfg, batch=1).sizes[4]
    sample_queries = min(queries, 21504)
    w = make_workload(cfg, batch=1, queries=sample_queries).to("cpu", dtype, loc_dtype)
    value, shapes, starts, loc, attn = w.operands(softmax=softmax)
    times = []
    for i in range(4):
        leaves = [t.detach().clone().requires_grad_(True) for t in (value, loc, attn)]
        t0 = time.perf_counter()
        out = eager_msda(leaves[0], shapes, starts, leaves[1], leaves[2], softmax=softmax)
        out.backward(w.grad_output)
        if i:
            times.append(time.perf_counter() - t0)
    full_pairs = cfg.batch * queries
    scale = full_pairs / (1 * sample_queries)
    return {
        "value": statistics.median(times) * 1e3 * scale,
        "unit": "ms/call",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (
            f"torch restatement of the reference eager backend (backends/eager/msda_pytorch.py) "
            f"fwd + autograd bwd, {str(dtype).split('.')[-1]}, batch 1 x {sample_queries} queries "
            f"of config {config} (1/{scale:g} of a call), median of 3 after 1 warm-up, scaled x{scale:g}; "
            f"host {os.cpu_count()} logical CPUs"
        ),
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=100)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--dtype", choices=sorted(DTYPES), default="bf16")
    parser.add_argument("--loc-dtype", choices=sorted(DTYPES), default=None)
    parser.add_argument("--method", choices=["linear", "softmax"], default="linear")
    parser.add_argument("--config", type=int, choices=sorted(CONFIGS), default=4)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument(
        "--copy-calibration", type=int, default=0, metavar="MIB",
        help="first run three plain device copies of MIB MiB, the known-size reference that "
             "scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters",
    )
    args = parser.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py measures one GPU: the MSDA op shards by batch or heads with no "
            "exchange, and this build runs on a single MI355X. "
            "Run it with --gpus 1.",
            file=sys.stderr,
        )
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2

    dtype = DTYPES[args.dtype]
    loc_dtype = DTYPES[args.loc_dtype] if args.loc_dtype else dtype
    softmax = args.method == "softmax"
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.copy_calibration > 0:
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.randn(n, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)  # one elementwise kernel: reads and writes MIB MiB
        torch.cuda.synchronize()
        del src, dst
    cfg = CONFIGS[args.config]
    w = make_workload(cfg).to(device, dtype, loc_dtype)
    B, S, H, D, Q, L, P = w.sizes
    es = torch.empty((), dtype=dtype).element_size()
    ls = torch.empty((), dtype=loc_dtype).element_size()
    fwd_bytes, bwd_bytes = algorithmic_bytes(B, S, H, D, Q, L, P, es, ls)

    ms_per_step, median_ms = time_fwd_bwd(w, args.steps, args.warmup, softmax)
    kernels = time_kernels(w, args.steps, args.warmup, softmax)
    bwd_gbs = bwd_bytes / (kernels["backward"] * 1e-3) / 1e9
    total_gbs = (fwd_bytes + bwd_bytes) / (ms_per_step * 1e-3) / 1e9

    profiled = args.config == 4 and args.dtype == "bf16" and loc_dtype == torch.bfloat16 and not softmax
    levels = "/".join(f"{h}x{w_}" for h, w_ in cfg.levels)
    queries = f"Q=S={S}" if cfg.queries is None else f"Q={Q}, S={S}"
    line = {
        "metric": METRIC,
        "value": round(ms_per_step, 5),
        "unit": "ms/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic",
        "config": {
            "workload": (
                f"config {args.config} {cfg.name}: B={B}, levels {levels}, {queries}, H={H}, D={D}, "
                f"P={P}, {args.dtype} value/weights, {str(loc_dtype).split('.')[-1]} locations, "
                f"{args.method} method, fwd+bwd via deformops_amd.registry.msda"
            ),
            "fwd_bwd_bytes": fwd_bytes + bwd_bytes,
            "fwd_bwd_achieved_gb_s": round(total_gbs, 1),
            "fwd_bwd_frac_of_hbm_peak": round(total_gbs / PEAK_HBM_GBS, 4),
            "median_ms_per_step": round(median_ms, 5),
            "forward_kernel_ms": round(kernels["forward"], 5),
            "backward_kernel_ms": round(kernels["backward"], 5),
            "forward_kernel_gb_s": round(fwd_bytes / (kernels["forward"] * 1e-3) / 1e9, 1),
            "device": torch.cuda.get_device_name(device),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "msda_backward (C-ABI call: bucket sort, softmax stats if softmax, grad_value, grad_sample)",
            "achieved": round(bwd_gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(bwd_gbs / PEAK_HBM_GBS, 4),
            "traffic": BACKWARD_TRAFFIC_BYTES if profiled else None,
            "algorithmic_bytes_per_launch": bwd_bytes,
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.config, dtype, loc_dtype, softmax)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
