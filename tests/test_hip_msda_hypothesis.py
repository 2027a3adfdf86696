"""Property-based parity of the HIP kernels with the CPU oracle over random shapes.

The GPU counterpart of the reference's hypothesis parity test
(``tests/deformops/test_msda_reference.py:31-88``), widened: batch, heads, head
width (odd ones included), levels and their shapes, points, queries, value dtype
(float64 included) and softmax / linear method are drawn together, and every example checks the forward and all three
gradients against the float64 C oracle with the tolerances of
``tests/test_hip_msda.py``. The owner kernel for grad_value (matrix cores or VALU)
and the bucket sort's counting mode (per-workgroup rows or atomics) are drawn too,
through the library's path override (msda_set_path_override). Examples are derandomized, so a GPU run
replays the same cases.
"""

from __future__ import annotations

import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from tests.test_hip_msda import BF16, F16, F32, F64, check_against_oracle
from tests.workloads import make_workload

pytestmark = pytest.mark.gpu

#: Kernel paths (msda_set_path_override bits): VALU owner kernel, atomic sort.
PATHS = {"default": 0, "valu": 1, "atomic-sort": 2, "valu-atomic-sort": 3}


@st.composite
def cases(draw):
    L = draw(st.integers(1, 5))
    levels = tuple((draw(st.integers(1, 40)), draw(st.integers(1, 40))) for _ in range(L))
    H = draw(st.sampled_from([1, 2, 3, 4, 8, 16]))
    D = draw(st.sampled_from([7, 8, 16, 24, 32, 48, 64]))
    return {
        "levels": levels,
        "batch": draw(st.integers(1, 3)),
        "queries": draw(st.integers(1, 300)),
        "heads": H,
        "channels": D,
        "points": draw(st.integers(1, 8)),
        "seed": draw(st.integers(0, 2**31 - 1)),
        "dtype": draw(st.sampled_from([F32, BF16, F16, F64])),
        "softmax": draw(st.booleans()),
        "path": draw(st.sampled_from(sorted(PATHS))),
    }


@given(case=cases())
@settings(max_examples=200, deadline=None, derandomize=True, database=None,
          suppress_health_check=[HealthCheck.too_slow, HealthCheck.data_too_large,
                                 HealthCheck.function_scoped_fixture])
def test_random_shapes_match_oracle(device, case):
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    with _lib.path_override(PATHS[case["path"]]):
        w = make_workload(0, levels=case["levels"], batch=case["batch"], queries=case["queries"],
                          heads=case["heads"], channels=case["channels"], points=case["points"],
                          seed=case["seed"]).to(device, case["dtype"])
        check_against_oracle(*w.operands(softmax=case["softmax"]), w.grad_output, softmax=case["softmax"],
                             dtype=case["dtype"], label=str(case))


@st.composite
def robustness_cases(draw):
    """The reference's backward robustness draws (``tests/deformops/test_msda_backward_robustness.py:29-77``):
    small random pyramids, locations far outside [0, 1] for half precision, and one
    query pushed to infinity."""
    L = draw(st.integers(1, 4))
    return {
        "levels": tuple((draw(st.integers(1, 32)), draw(st.integers(1, 32))) for _ in range(L)),
        "batch": draw(st.integers(1, 2)),
        "heads": draw(st.sampled_from([1, 2, 4])),
        "channels": draw(st.sampled_from([8, 16, 32])),
        "points": draw(st.sampled_from([1, 2, 4, 8])),
        "queries": draw(st.integers(1, 128)),
        "dtype": draw(st.sampled_from([F32, F16, BF16])),
        "seed": draw(st.integers(0, 2**31 - 1)),
        "infinite_query": draw(st.one_of(st.none(), st.integers(0, 127))),
        "softmax": draw(st.booleans()),
    }


@given(case=robustness_cases())
@settings(max_examples=100, deadline=None, derandomize=True, database=None,
          suppress_health_check=[HealthCheck.too_slow, HealthCheck.data_too_large,
                                 HealthCheck.function_scoped_fixture])
def test_backward_stays_finite(device, case):
    """Every gradient is finite, for every query: the kernels skip samples with a
    non-finite location (zero contribution, zero gradient), where the reference only
    asks finiteness of the other queries' gradients."""
    from deformops_amd.registry import msda  # noqa: PLC0415

    dtype = case["dtype"]
    w = make_workload(0, levels=case["levels"], batch=case["batch"], queries=case["queries"],
                      heads=case["heads"], channels=case["channels"], points=case["points"],
                      seed=case["seed"])
    value, shapes, starts, loc, attn = w.operands(softmax=case["softmax"])
    if dtype != F32:
        value = value * 1e-2
        loc = (loc * 2 - 1) * 10.0
    if case["infinite_query"] is not None:
        loc = loc.clone()
        loc[:, case["infinite_query"] % loc.shape[1]] = float("inf")
    leaves = [t.to(device, dtype).requires_grad_(True) for t in (value, loc, attn)]
    out = msda(leaves[0], shapes.to(device), starts.to(device), leaves[1], leaves[2],
               method="softmax" if case["softmax"] else "linear")
    out.float().sum().backward()
    assert torch.isfinite(out).all()
    for leaf in leaves:
        assert leaf.grad is not None and torch.isfinite(leaf.grad).all()
