"""Benchmark of the MI355X MSDA kernels on the BASELINE headline workload.

One step = one forward and one backward of ``deformops_amd.registry.msda`` on
config 4 (Mask2Former pixel-decoder encoder, large): B=4, levels 128x128, 64x64,
32x32 (Q = S = 21,504), H=8, D=32, P=4, bfloat16 value, weights and locations,
linear method, synthetic seeded inputs already resident in HBM.

Prints one JSON line. ``value`` is fwd+bwd milliseconds per call through the
public API (lower is better), timed over exactly ``--steps`` steps after
``--warmup`` untimed ones. Before anything is timed the GPU runs the workload's
C-ABI fwd+bwd pair, untimed, for 0.3 s (``config.untimed_settle``), so that its
clocks have left the idle state, and before the public-API steps it runs those
steps, untimed, for another 0.3 s (fresh allocator blocks are slower at first).
``roofline`` rates one fwd+bwd pair of C-ABI calls (msda_forward, then
msda_backward_workspace as the autograd bridge calls it, back to back on one stream,
bracketed by HIP events on that stream) by its algorithmic bytes against 8 TB/s;
``roofline.backward_call`` rates the backward call alone, and ``roofline.gather``
rates the forward kernel's corner gathers against the random-row gather rate of
L1 and L2 that the row-gather probe (libmsda_probe.so) measures in the same run
(``l2_peak_128b_rows``: the same probe with 128-byte rows, whole cache lines).
``roofline.l2_requests`` rates the forward, grad_value and grad_sample kernels by
L2 requests per second, the quantity that bounds the gathers: each one's request
count per launch from the counter pass in profiles/msda_config4_bf16_l2_requests.md
(when that pass ran on the kernel and probe sources being measured) over its live
time in this run (the forward call; the backward's phases, timed by HIP events the
library records between them, msda_set_phase_events), against the probe's.
``roofline.traffic`` is the HBM bytes of one fwd+bwd from the rocprofv3 counter
passes in profiles/msda_config4_bf16_hbm_traffic.md, reported only when those
passes ran on the kernel source being measured. ``cpu_baseline`` times the torch
restatement of the reference's eager CPU path on a bounded sample of the same
workload, scaled to one full call, on all physical cores.

    python bench.py [--steps K] [--warmup W] [--dtype bf16|f16|f32] [--loc-dtype ...]
                    [--method linear|softmax] [--config 0..4] [--grad-value owner|atomic]

``--config`` measures another BASELINE configuration the same way (config 4 is the
headline and the only one the driver's line is quoted on). ``--grad-value atomic``
runs the backward's grad_value with global atomics (MSDA_GRAD_VALUE_ATOMIC) in the
C-ABI timings, for comparison with the owner-computes default.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import re
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
DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
KERNEL_SOURCE = REPO / "deformops_amd" / "csrc" / "msda.hip"
TRAFFIC_PROFILE = REPO / "profiles" / "msda_config4_bf16_hbm_traffic.md"
PROBE_SOURCE = REPO / "bench_probe" / "gather_probe.hip"
REQUEST_PROFILE = REPO / "profiles" / "msda_config4_bf16_l2_requests.md"
PROBE_BYTES = 2048 * 256 * 128 * 8 * 16  # bytes one probe launch gathers (see row_gather_rates)
SETTLE_S = 0.3  # untimed seconds of the measured work before each timing (see settle_clocks)
CPU_WARMUP, CPU_TIMED = 2, 5  # iterations of the CPU baseline


def _events(n: int) -> list[torch.cuda.Event]:
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def time_fwd_bwd(w, steps: int, warmup: int, softmax: bool, settle_s: float = SETTLE_S):
    """Time K full fwd+bwd steps through the public API; wall clock and per-step events.

    First, untimed, the same step for ``settle_s`` seconds: a process's first ~50
    steps through the public API run up to 8 % slower on the GPU (fresh
    caching-allocator blocks for the outputs and gradients), with the clocks
    already settled; then the W warm-up steps and the K timed ones.
    """
    from deformops_amd.registry import msda  # noqa: PLC0415

    value, shapes, starts, loc, attn = w.operands(softmax=softmax)
    leaves = [t.detach().clone().requires_grad_(True) for t in (value, loc, attn)]
    method = "softmax" if softmax else "linear"

    def step() -> None:
        for leaf in leaves:
            leaf.grad = None
        out = msda(leaves[0], shapes, starts, leaves[1], leaves[2], method=method)
        out.backward(w.grad_output)

    t_settle = time.perf_counter()
    while time.perf_counter() - t_settle < settle_s:
        for _ in range(10):
            step()
        torch.cuda.synchronize()
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


def settle_clocks(w, softmax: bool, seconds: float = SETTLE_S) -> dict[str, float]:
    """Untimed: the workload's C-ABI fwd+bwd pair, repeated until ``seconds`` have passed.

    An MI355X that has been idle runs its first ~0.1 s of work at lower clocks: with
    5 warm-up steps the timed steps measure 0.52 ms where 100 warm-up steps give
    0.49 ms. So before anything is timed the GPU runs the measured work itself until
    its clocks have settled.
    """
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    lib = _lib.load()
    value, shapes, starts, loc, attn = w.operands(softmax=softmax)
    B, S, H, D, Q, L, P = w.sizes
    out = torch.empty((B, Q, H * D), dtype=value.dtype, device=value.device)
    gv, gl, ga = torch.empty_like(value), torch.empty_like(loc), torch.empty_like(attn)
    stream = torch.cuda.current_stream().cuda_stream
    flags = _lib.FLAG_SOFTMAX if softmax else 0
    ws = torch.empty(lib.workspace_size(value.dtype, B, S, H, D, Q, L, P, flags), dtype=torch.uint8,
                     device=value.device)
    vcode, lcode = _lib.DTYPE_CODES[value.dtype], _lib.DTYPE_CODES[loc.dtype]
    icode = _lib.INDEX_CODES[shapes.dtype]
    t0, calls = time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            lib.check(lib.forward(value.data_ptr(), vcode, shapes.data_ptr(), starts.data_ptr(), icode,
                                  loc.data_ptr(), lcode, attn.data_ptr(), out.data_ptr(),
                                  B, S, H, D, Q, L, P, flags, stream))
            lib.check(lib.backward_workspace(value.data_ptr(), vcode, shapes.data_ptr(), starts.data_ptr(), icode,
                                             loc.data_ptr(), lcode, attn.data_ptr(), w.grad_output.data_ptr(),
                                             gv.data_ptr(), gl.data_ptr(), ga.data_ptr(),
                                             B, S, H, D, Q, L, P, flags, ws.data_ptr(), ws.numel(), stream))
        calls += 10
        torch.cuda.synchronize()
    return {"settle_s": round(time.perf_counter() - t0, 3), "settle_pairs": calls}


def time_calls(w, steps: int, warmup: int, softmax: bool, bwd_flags: int) -> dict[str, float]:
    """Average device time of the C-ABI calls on torch's current stream: the forward
    (one kernel), the backward (the bucket sort, the softmax statistics, grad_value,
    grad_sample), and a forward then a backward back to back."""
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    lib = _lib.load()
    value, shapes, starts, loc, attn = w.operands(softmax=softmax)
    B, S, H, D, Q, L, P = w.sizes
    out = torch.empty((B, Q, H * D), dtype=value.dtype, device=value.device)
    gv, gl, ga = torch.empty_like(value), torch.empty_like(loc), torch.empty_like(attn)
    stream = torch.cuda.current_stream()
    flags = _lib.FLAG_SOFTMAX if softmax else 0
    # The workspace entry point, as the autograd bridge calls it (grad_sample beside the
    # sort, except while the phase events are set: then the kernels run in turn).
    ws = torch.empty(lib.workspace_size(value.dtype, B, S, H, D, Q, L, P, flags), dtype=torch.uint8,
                     device=value.device)
    vcode, lcode = _lib.DTYPE_CODES[value.dtype], _lib.DTYPE_CODES[loc.dtype]
    icode = _lib.INDEX_CODES[shapes.dtype]

    def fwd() -> None:
        lib.check(lib.forward(value.data_ptr(), vcode, shapes.data_ptr(), starts.data_ptr(), icode,
                              loc.data_ptr(), lcode, attn.data_ptr(), out.data_ptr(),
                              B, S, H, D, Q, L, P, flags, stream.cuda_stream))

    def bwd() -> None:
        lib.check(lib.backward_workspace(value.data_ptr(), vcode, shapes.data_ptr(), starts.data_ptr(), icode,
                                         loc.data_ptr(), lcode, attn.data_ptr(), w.grad_output.data_ptr(),
                                         gv.data_ptr(), gl.data_ptr(), ga.data_ptr(),
                                         B, S, H, D, Q, L, P, flags | bwd_flags, ws.data_ptr(), ws.numel(),
                                         stream.cuda_stream))

    def both() -> None:
        fwd()
        bwd()

    result = {}
    # The backward's phases (bucket sort, grad_value, grad_sample), from the events the
    # library records between them (msda_set_phase_events), in their own loop so that
    # the recording stays out of the other timings.
    marks = _events(4)
    for ev in marks:
        ev.record(stream)
    torch.cuda.synchronize()
    lib.set_phase_events([ev.cuda_event for ev in marks])
    phases: dict[str, list[float]] = {"sort": [], "grad_value": [], "grad_sample": []}
    try:
        for i in range(warmup + steps):
            bwd()
            marks[3].synchronize()
            if i >= warmup:
                for k, name in enumerate(phases):
                    phases[name].append(marks[k].elapsed_time(marks[k + 1]))
    finally:
        lib.set_phase_events(None)
    for name, times in phases.items():
        result["phase_" + name] = statistics.mean(times)
    for name, fn in (("forward", fwd), ("backward", bwd), ("fwd_bwd", both)):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        marks = []
        for _ in range(steps):
            s, e = _events(2)
            s.record(stream)
            fn()
            e.record(stream)
            marks.append((s, e))
        torch.cuda.synchronize()
        result[name] = statistics.mean(s.elapsed_time(e) for s, e in marks)
    return result


def row_gather_rates(device: torch.device) -> dict[str, float]:
    """GB/s of random 64-byte row gathers (4 lanes x 16 bytes each) from a 16 KiB buffer
    (L1-resident on every CU) and a 2 MiB one (L2-resident on every XCD), and of
    random 128-byte rows (8 lanes, one cache line each) from the 2 MiB buffer, from
    the probe kernel of bench_probe/libmsda_probe.so; mean of 5 launches of 2048 x 256 threads."""
    import ctypes  # noqa: PLC0415

    path = REPO / "bench_probe" / "libmsda_probe.so"
    probe = ctypes.CDLL(str(path))
    probe.msda_probe_row_gather.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    probe.msda_probe_row_gather.restype = ctypes.c_int
    blocks, iters, threads = 2048, 128, 256
    sink = torch.empty(blocks * threads, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream()
    rates = {}
    for name, nbytes, row_bytes in (("l1", 16 << 10, 64), ("l2", 2 << 20, 64), ("l2_128", 2 << 20, 128)):
        buf = torch.randint(0, 1 << 30, (nbytes // 4,), dtype=torch.int32, device=device)
        rows = nbytes // row_bytes

        def launch() -> None:
            rc = probe.msda_probe_row_gather(buf.data_ptr(), rows, row_bytes, blocks, iters, sink.data_ptr(),
                                             stream.cuda_stream)
            if rc != 0:
                raise RuntimeError("row-gather probe launch failed")

        for _ in range(2):
            launch()
        times = []
        for _ in range(5):
            s, e = _events(2)
            s.record(stream)
            launch()
            e.record(stream)
            e.synchronize()
            times.append(s.elapsed_time(e))
        gathered = blocks * threads * iters * 8 * 16  # lanes x loads x 16 bytes
        rates[name] = gathered / (statistics.mean(times) * 1e-3) / 1e9
    return rates


def profiled_traffic() -> tuple[int | None, str]:
    """HBM bytes of one fwd+bwd of the default workload, from the counter passes in
    profiles/, when they ran on this kernel source; else ``None`` and why."""
    if not TRAFFIC_PROFILE.exists():
        return None, "no counter profile committed"
    text = TRAFFIC_PROFILE.read_text()
    sha = re.search(r"kernel_source_sha256:\s*([0-9a-f]{64})", text)
    total = re.search(r"traffic_bytes_per_fwd_bwd:\s*(\d+)", text)
    if not sha or not total:
        return None, "the counter profile states no source hash or total"
    current = hashlib.sha256(KERNEL_SOURCE.read_bytes()).hexdigest()
    if sha.group(1) != current:
        return None, "the counter profile was taken on another kernel source"
    return int(total.group(1)), f"rocprofv3 FETCH_SIZE x2 + WRITE_SIZE passes, {TRAFFIC_PROFILE.relative_to(REPO)}"


def profiled_l2_requests() -> tuple[dict[str, int] | None, str]:
    """L2 requests per launch of the MSDA kernels and of the 2 MiB, 64-byte-row probe
    at the default workload, from the counter pass in profiles/, when it ran on these
    kernel and probe sources; else ``None`` and why."""
    if not REQUEST_PROFILE.exists():
        return None, "no request profile committed"
    text = REQUEST_PROFILE.read_text()
    shas = dict(re.findall(r"(kernel|probe)_source_sha256:\s*([0-9a-f]{64})", text))
    counts = {name: int(n) for name, n in re.findall(r"l2_requests_per_launch (\S+):\s*(\d+)", text)}
    if "kernel" not in shas or "probe" not in shas or "msda_forward_kernel" not in counts or "probe_l2" not in counts:
        return None, "the request profile states no source hashes or counts"
    for key, path in (("kernel", KERNEL_SOURCE), ("probe", PROBE_SOURCE)):
        if shas[key] != hashlib.sha256(path.read_bytes()).hexdigest():
            return None, f"the request profile was taken on another {key} source"
    return counts, f"rocprofv3 TCC_HIT_sum + TCC_MISS_sum pass, {REQUEST_PROFILE.relative_to(REPO)}"


def host_cpu() -> dict:
    """The host's CPU model, logical CPUs and physical cores (from /proc/cpuinfo)."""
    model, cores = "unknown", set()
    try:
        phys = core = None
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            key, _, val = (part.strip() for part in line.partition(":"))
            if key == "model name":
                model = val
            elif key == "physical id":
                phys = val
            elif key == "core id":
                core = val
            elif not line.strip() and core is not None:
                cores.add((phys, core))
                phys = core = None
    except OSError:
        pass
    logical = os.cpu_count() or 1
    return {"model": model, "logical_cpus": logical, "physical_cores": len(cores) or logical}


def cpu_baseline(config: int, dtype: torch.dtype, loc_dtype: torch.dtype, softmax: bool) -> dict:
    """The reference's eager CPU path (torch restatement) on a bounded sample, on all
    physical cores: in the workload's dtype, and in float32 too when that differs
    (the CPU accumulates 16-bit dtypes in 16 bits).

    Sample: batch 1 and at most the first 21,504 queries of the configuration (at
    config 4, one image: 21,504 of the 86,016 (batch, query) pairs); 2 warm-up and 5
    timed fwd + autograd-bwd iterations, median, scaled by the call's (batch, query)
    pairs over the sample's.
    """
    from oracle.eager import eager_msda  # noqa: PLC0415

    cpu = host_cpu()
    threads_before = torch.get_num_threads()
    torch.set_num_threads(cpu["physical_cores"])
    cfg = CONFIGS[config]
    full_queries = cfg.queries if cfg.queries is not None else sum(h * w for h, w in cfg.levels)
    sample_queries = min(full_queries, 21504)
    base = make_workload(cfg, batch=1, queries=sample_queries)

    def median_ms(dt: torch.dtype, lt: torch.dtype) -> float:
        w = base.to("cpu", dt, lt)
        value, shapes, starts, loc, attn = w.operands(softmax=softmax)
        times = []
        for i in range(CPU_WARMUP + CPU_TIMED):
            leaves = [t.detach().clone().requires_grad_(True) for t in (value, loc, attn)]
            t0 = time.perf_counter()
            out = eager_msda(leaves[0], shapes, starts, leaves[1], leaves[2], softmax=softmax)
            out.backward(w.grad_output)
            if i >= CPU_WARMUP:
                times.append(time.perf_counter() - t0)
        return statistics.median(times) * 1e3

    scale = cfg.batch * full_queries / sample_queries
    try:
        value_ms = median_ms(dtype, loc_dtype) * scale
        f32_ms = value_ms if dtype == torch.float32 else median_ms(torch.float32, torch.float32) * scale
    finally:
        torch.set_num_threads(threads_before)
    name = str(dtype).split(".")[-1]
    return {
        "value": round(value_ms, 2),
        "unit": "ms/call",
        "cores": cpu["physical_cores"],
        "kind": "port",
        "value_float32": round(f32_ms, 2),
        "cpu": cpu,
        "sample": (
            f"torch restatement of the reference eager backend (backends/eager/msda_pytorch.py) "
            f"fwd + autograd bwd, {name} (and float32 for value_float32), batch 1 x {sample_queries} queries "
            f"of config {config} (1/{scale:g} of a call), median of {CPU_TIMED} after {CPU_WARMUP} warm-up, "
            f"scaled x{scale:g}; "
            f"torch.set_num_threads({cpu['physical_cores']}) on {cpu['model']}"
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
    parser.add_argument("--grad-value", choices=["owner", "atomic"], default="owner")
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
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    cfg = CONFIGS[args.config]
    w = make_workload(cfg).to(device, dtype, loc_dtype)
    B, S, H, D, Q, L, P = w.sizes
    es = torch.empty((), dtype=dtype).element_size()
    ls = torch.empty((), dtype=loc_dtype).element_size()
    fwd_bytes, bwd_bytes = algorithmic_bytes(B, S, H, D, Q, L, P, es, ls)
    bwd_flags = _lib.FLAG_GRAD_VALUE_ATOMIC if args.grad_value == "atomic" else 0

    settled = settle_clocks(w, softmax)
    calls = time_calls(w, args.steps, args.warmup, softmax, bwd_flags)
    gather = row_gather_rates(device)
    ms_per_step, median_ms = time_fwd_bwd(w, args.steps, args.warmup, softmax)

    total_gbs = (fwd_bytes + bwd_bytes) / (ms_per_step * 1e-3) / 1e9
    call_gbs = (fwd_bytes + bwd_bytes) / (calls["fwd_bwd"] * 1e-3) / 1e9
    bwd_gbs = bwd_bytes / (calls["backward"] * 1e-3) / 1e9
    corner_bytes = B * Q * H * L * P * 4 * D * es  # every sample loads 4 corner rows
    corner_gbs = corner_bytes / (calls["forward"] * 1e-3) / 1e9
    default = args.config == 4 and args.dtype == "bf16" and loc_dtype == torch.bfloat16 and not softmax
    traffic, traffic_source = profiled_traffic() if default and args.grad_value == "owner" else (
        None, "profiled for the default workload only")
    requests, request_source = profiled_l2_requests() if default else (None, "profiled for the default workload only")
    l2_requests: dict = {"kernel": "msda_forward_kernel", "source": request_source}
    if requests is not None:
        # Requests per second: each kernel's profiled count over its live time (the
        # forward call, and the backward's grad_value and grad_sample phases), and the
        # probe's profiled count over its live launch time (from its GB/s).
        peak = requests["probe_l2"] / (PROBE_BYTES / (gather["l2"] * 1e9)) / 1e9
        live = {"msda_forward_kernel": calls["forward"], "msda_grad_value_mfma_kernel": calls["phase_grad_value"],
                "msda_grad_sample_kernel": calls["phase_grad_sample"]}
        kernels = {}
        for kernel, ms in live.items():
            if kernel in requests:
                achieved = requests[kernel] / (ms * 1e-3) / 1e9
                kernels[kernel] = {"requests_per_launch": requests[kernel], "ms": round(ms, 5),
                                   "achieved": round(achieved, 1), "frac": round(achieved / peak, 4)}
        forward = kernels["msda_forward_kernel"]
        l2_requests.update({"requests_per_launch": forward["requests_per_launch"], "achieved": forward["achieved"],
                            "peak": round(peak, 1), "unit": "G requests/s", "frac": forward["frac"],
                            "kernels": kernels,
                            "peak_source": "the 2 MiB 64-byte-row probe of this run (one L2 request per row)"})

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
            "grad_value": args.grad_value,
            "fwd_bwd_bytes": fwd_bytes + bwd_bytes,
            "fwd_bwd_achieved_gb_s": round(total_gbs, 1),
            "fwd_bwd_frac_of_hbm_peak": round(total_gbs / PEAK_HBM_GBS, 4),
            "median_ms_per_step": round(median_ms, 5),
            "forward_call_ms": round(calls["forward"], 5),
            "backward_call_ms": round(calls["backward"], 5),
            "backward_phase_ms": {name: round(calls["phase_" + name], 5)
                                  for name in ("sort", "grad_value", "grad_sample")},
            "untimed_settle": settled,
            "device": torch.cuda.get_device_name(device),
        },
        "roofline": {
            # The contract's roofline is HBM bandwidth (the op is a gather / scatter:
            # no MFMA-bound formulation). The limit the kernels meet below it is the L2
            # request rate of their row gathers (forward, grad_sample) and the latency
            # of grad_value's scattered candidate reads: "binding" and "l2_requests".
            "bound": "hbm",
            "binding": "l2_request_rate (forward, grad_sample); memory latency (grad_value)",
            "kernel": "one msda_forward + msda_backward_workspace C-ABI call pair (forward kernel, bucket sort, "
                      "grad_value, grad_sample beside the sort on a side stream), on one caller stream",
            "achieved": round(call_gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(call_gbs / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "algorithmic_bytes_per_launch": fwd_bytes + bwd_bytes,
            "launch_ms": round(calls["fwd_bwd"], 5),
            "backward_call": {
                "algorithmic_bytes": bwd_bytes,
                "ms": round(calls["backward"], 5),
                "achieved": round(bwd_gbs, 1),
                "frac": round(bwd_gbs / PEAK_HBM_GBS, 4),
            },
            "gather": {
                "kernel": "msda_forward_kernel: 4 corner rows of D channels per sample",
                "bytes": corner_bytes,
                "achieved": round(corner_gbs, 1),
                "l1_peak": round(gather["l1"], 1),
                "l2_peak": round(gather["l2"], 1),
                "l2_peak_128b_rows": round(gather["l2_128"], 1),
                "unit": "GB/s",
                "frac_of_l2": round(corner_gbs / gather["l2"], 4),
                "frac_of_l1": round(corner_gbs / gather["l1"], 4),
                "peak_source": "random 64-byte row gathers from a 2 MiB (L2) and 16 KiB (L1) buffer, "
                               "and 128-byte rows from the 2 MiB buffer, libmsda_probe.so, this run",
            },
            "l2_requests": l2_requests,
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.config, dtype, loc_dtype, softmax)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
