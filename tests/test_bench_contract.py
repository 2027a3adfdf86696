"""The parts of bench.py's command-line contract that need no GPU: more than one GPU
is refused with a message and exit status 2, every BASELINE configuration is
accepted, and the CPU baseline's sample is bounded and scaled to one full call.
"""

from __future__ import annotations

import json
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parent.parent


def run_bench(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(REPO / "bench.py"), *args], capture_output=True, text=True,
                          timeout=300, cwd=REPO, check=False)


def test_more_than_one_gpu_is_refused():
    result = run_bench("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert result.returncode == 2
    assert "one GPU" in result.stderr
    assert result.stdout == ""


def test_unknown_config_is_a_usage_error():
    result = run_bench("--config", "7")
    assert result.returncode == 2
    assert "invalid choice" in result.stderr


def test_cpu_baseline_of_the_small_configuration():
    sys.path.insert(0, str(REPO))
    import bench  # noqa: PLC0415

    line = bench.cpu_baseline(0, torch.float32, torch.float32, softmax=False)
    assert line["unit"] == "ms/call" and line["kind"] == "port" and line["value"] > 0
    assert "config 0" in line["sample"] and "(1/1 of a call)" in line["sample"]
    json.dumps(line)


@pytest.mark.parametrize("config", [1, 4])
def test_cpu_baseline_sample_is_bounded(config, monkeypatch):
    """The sample is batch 1 and at most 21,504 queries; the value is scaled by the
    call's (batch, query) pairs over the sample's."""
    sys.path.insert(0, str(REPO))
    import bench  # noqa: PLC0415

    samples = []
    make = bench.make_workload

    def tiny_sample(cfg, **kwargs):  # noqa: ANN001, ANN003
        if "queries" in kwargs:  # the timed sample: record it, run it on a small pyramid
            samples.append((kwargs["batch"], kwargs["queries"]))
            kwargs = {**kwargs, "levels": ((4, 4),), "queries": 8}
        return make(cfg, **kwargs)

    monkeypatch.setattr(bench, "make_workload", tiny_sample)
    line = bench.cpu_baseline(config, torch.float32, torch.float32, softmax=False)
    cfg = bench.CONFIGS[config]
    queries = 300 if config == 1 else 21504
    assert samples == [(1, min(queries, 21504))]
    assert f"x{cfg.batch * queries / min(queries, 21504):g}" in line["sample"]


def test_committed_request_profile_parses():
    """profiles/msda_config4_bf16_l2_requests.md carries the forward's and the probe's
    L2 request counts and the source hashes they were taken on. bench.py reports the
    counts only while those hashes match the tree (else ``None`` and the reason)."""
    import bench  # noqa: PLC0415

    text = bench.REQUEST_PROFILE.read_text()
    assert re.search(r"kernel_source_sha256:\s*[0-9a-f]{64}", text)
    assert re.search(r"probe_source_sha256:\s*[0-9a-f]{64}", text)
    counts = {name: int(n) for name, n in re.findall(r"l2_requests_per_launch (\S+):\s*(\d+)", text)}
    assert counts["msda_forward_kernel"] > 0 and counts["probe_l2"] > counts["probe_l2_128"] > 0
    found, source = bench.profiled_l2_requests()
    assert found == counts or (found is None and "another" in source), source
