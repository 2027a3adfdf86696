"""The CPU backend (``Backend.EAGER``, deformops_amd/backends/eager/msda.py) against
the float64 C oracle, through ``registry.msda`` and autograd.

The reference's CPU tensors run its eager backend (registry/msda.py:204-205); its
tests compare that backend with ``grid_sample`` and on known answers
(tests/deformops/test_msda_eager.py:36-212). Here the same cases run against the
oracle, which those checks pin (tests/test_oracle.py). Tolerances, norm-wise:
float64 1e-12, float32 1e-5, 16-bit 2e-2 (the operands are rounded once; the
backend computes in float32). CPU only: GPU tensors never take this backend.
"""

from __future__ import annotations

import math

import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

import oracle
from deformops_amd.core.errors import NoBackendError
from deformops_amd.registry import Backend, MSDAContext, msda, select_backend
from tests.workloads import make_workload

F32, BF16, F16, F64 = torch.float32, torch.bfloat16, torch.float16, torch.float64
TOL = {F64: 1e-12, F32: 1e-5, BF16: 2e-2, F16: 2e-2}


def rel_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    actual = actual.detach().to(F64).reshape(expected.shape)
    scale = expected.abs().max().item()
    diff = (actual - expected).abs().max().item()
    return diff / scale if scale else diff


def run(value, shapes, starts, loc, attn, grad_output, *, softmax, backend=None):
    leaves = [t.detach().clone().requires_grad_(True) for t in (value, loc, attn)]
    out = msda(leaves[0], shapes, starts, leaves[1], leaves[2], method="softmax" if softmax else "linear",
               backend=backend)
    out.backward(grad_output)
    return out.detach(), leaves[0].grad, leaves[1].grad, leaves[2].grad


def check(value, shapes, starts, loc, attn, grad_output, *, softmax, dtype, label=""):
    got = run(value, shapes, starts, loc, attn, grad_output, softmax=softmax)
    assert got[0].dtype == value.dtype
    assert got[1].dtype == value.dtype and got[2].dtype == loc.dtype and got[3].dtype == attn.dtype
    expected = (oracle.forward(value, shapes, starts, loc, attn, softmax=softmax),
                *oracle.backward(value, shapes, starts, loc, attn, grad_output, softmax=softmax))
    names = ("output", "grad_value", "grad_loc", "grad_attn")
    errs = {n: rel_err(g, e) for n, g, e in zip(names, got, expected, strict=True)}
    bad = {n: e for n, e in errs.items() if not e <= TOL[dtype]}
    assert not bad, f"{label} softmax={softmax}: {errs} exceed {TOL[dtype]}"


SHAPES = [
    # (levels, B, Q, H, D, P)
    pytest.param(((8, 8), (4, 4), (2, 2)), 2, 12, 4, 32, 4, id="three-levels"),
    pytest.param(((1, 1),), 3, 4, 2, 16, 1, id="1x1-level"),
    pytest.param(((1, 7), (6, 1), (1, 1)), 1, 9, 3, 8, 4, id="one-row-one-column"),
    pytest.param(((6, 9), (3, 5)), 2, 7, 3, 24, 3, id="odd-heads-d24-p3"),
    pytest.param(((5, 5),), 1, 6, 2, 7, 2, id="d7"),
    pytest.param(((10, 12), (5, 6), (3, 3), (2, 2), (1, 1)), 1, 9, 2, 64, 8, id="five-levels-p8"),
]


@pytest.mark.parametrize("dtype", [F64, F32, BF16, F16], ids=["f64", "f32", "bf16", "f16"])
@pytest.mark.parametrize(("levels", "B", "Q", "H", "D", "P"), SHAPES)
def test_shapes_match_oracle(levels, B, Q, H, D, P, dtype):
    w = make_workload(0, levels=levels, batch=B, queries=Q, heads=H, channels=D, points=P, seed=Q + D)
    w = w.to("cpu", dtype)
    for softmax in (False, True):
        check(*w.operands(softmax=softmax), w.grad_output, softmax=softmax, dtype=dtype, label=str(levels))


@pytest.mark.parametrize(("dtype", "loc_dtype"), [(F32, F32), (BF16, F32)], ids=["f32", "bf16-f32loc"])
def test_config_0_matches_oracle(dtype, loc_dtype):
    """BASELINE config 0, the reference's own CPU-runnable case, at full size."""
    w = make_workload(0).to("cpu", dtype, loc_dtype)
    for softmax in (False, True):
        check(*w.operands(softmax=softmax), w.grad_output, softmax=softmax, dtype=dtype, label="config 0")


def test_overlapping_and_malformed_levels():
    """Levels sharing positions of S sum into shared grad_value elements; a level
    that does not fit S contributes nothing (the kernels' reading of such tables)."""
    g = torch.Generator().manual_seed(3)
    B, Q, H, D, P, S = 2, 11, 2, 8, 4, 30
    value = torch.randn(B, S, H, D, generator=g, dtype=F64)
    loc = torch.rand(B, Q, H, 3, P, 2, generator=g, dtype=F64) * 1.1 - 0.05
    attn = torch.rand(B, Q, H, 3 * P, generator=g, dtype=F64)
    grad = torch.randn(B, Q, H * D, generator=g, dtype=F64)
    shapes = torch.tensor([[6, 5], [4, 4], [5, 4]])
    for starts in (torch.tensor([0, 10, 0]), torch.tensor([0, 10, 12])):  # the last: 12 + 20 > S
        for softmax in (False, True):
            check(value, shapes, starts, loc, attn, grad, softmax=softmax, dtype=F64, label=str(starts.tolist()))


def test_pixel_boundaries_and_out_of_bounds():
    """Samples at -1 <= x < W count (x = -1 only through its right corner); samples
    outside, and non-finite ones, give zero output and zero location gradients."""
    shapes, starts = torch.tensor([[3, 4]]), torch.tensor([0])
    value = torch.arange(12 * 2, dtype=F64).reshape(1, 12, 1, 2)
    W, Hh = 4, 3
    xs = [(-1 + 0.5) / W, (-0.5 + 0.5) / W, (3.0 + 0.5) / W, (3.999 + 0.5) / W, (4.0 + 0.5) / W,
          -2.0, 5.0, math.inf, -math.inf, math.nan]
    loc = torch.tensor([[x, (1.0 + 0.5) / Hh] for x in xs], dtype=F64).reshape(1, len(xs), 1, 1, 1, 2)
    attn = torch.ones(1, len(xs), 1, 1, dtype=F64)
    grad = torch.ones(1, len(xs), 2, dtype=F64)
    out, gv, gl, ga = run(value, shapes, starts, loc, attn, grad, softmax=False)
    finite = loc.clone()
    finite[~torch.isfinite(finite)] = 7.0  # the oracle takes finite locations; 7 is outside too
    assert rel_err(out, oracle.forward(value, shapes, starts, finite, attn)) <= 1e-12
    expected = oracle.backward(value, shapes, starts, finite, attn, grad)
    for got, want in zip((gv, gl, ga), expected, strict=True):
        assert rel_err(got, want) <= 1e-12
    assert out[0, 4:].abs().max() == 0 and gl[0, 4:].abs().max() == 0
    assert torch.isfinite(gv).all() and torch.isfinite(gl).all() and torch.isfinite(ga).all()


def test_softmax_with_negative_infinite_logit():
    w = make_workload(0, levels=((4, 4),), batch=1, queries=3, heads=2, channels=8, points=4).to("cpu", F64)
    value, shapes, starts, loc, logits = w.operands(softmax=True)
    logits = logits.clone()
    logits[0, 0, 0, 1] = -math.inf
    check(value, shapes, starts, loc, logits, w.grad_output, softmax=True, dtype=F64)


def test_split_weights_and_int32_tables():
    w = make_workload(0, levels=((6, 6), (3, 3)), batch=1, queries=7, heads=2, channels=8).to("cpu", F32)
    value, shapes, starts, loc, attn = w.operands()
    split = attn.reshape(*attn.shape[:3], 2, -1)
    flat = msda(value, shapes, starts, loc, attn)
    torch.testing.assert_close(msda(value, shapes.int(), starts.int(), loc, split), flat, rtol=0, atol=0)


@pytest.mark.parametrize("softmax", [False, True], ids=["linear", "softmax"])
def test_float64_gradcheck(softmax):
    w = make_workload(0, levels=((4, 5), (2, 2)), batch=1, queries=3, heads=2, channels=4, points=2,
                      locations="uniform").to("cpu", F64)
    value, shapes, starts, loc, attn = w.operands(softmax=softmax)
    method = "softmax" if softmax else "linear"
    torch.autograd.gradcheck(lambda v, lc, a: msda(v, shapes, starts, lc, a, method=method),
                             (value.requires_grad_(), loc.requires_grad_(), attn.requires_grad_()),
                             eps=1e-6, atol=1e-5)


def test_compiled_call_matches_eager():
    """The public operator traces on the CPU: the backend uses tensor operations only."""
    w = make_workload(0, levels=((6, 6), (3, 3)), batch=1, queries=7, heads=2, channels=8).to("cpu", F32)
    ops = w.operands()
    compiled = torch.compile(lambda *a: msda(*a), backend="aot_eager", fullgraph=True)
    torch.testing.assert_close(compiled(*ops), msda(*ops), rtol=0, atol=0)


def test_policy_keeps_gpu_tensors_off_the_cpu_backend():
    """select_backend sends CPU contexts to EAGER and GPU contexts to HIP alone; the
    eager backend declines a GPU context, so a GPU call can never land on it."""
    from deformops_amd.backends.eager.msda import supports_context  # noqa: PLC0415

    def context(device: str) -> MSDAContext:
        return MSDAContext(device=torch.device(device), num_levels=3, num_heads=8, num_points=4,
                           dtype=BF16, sm_version=(0, 0), is_training=True, num_queries=10, head_dim=32)

    assert select_backend(context("cpu")) == [Backend.EAGER]
    assert select_backend(context("cuda")) == [Backend.HIP]
    assert supports_context(context("cpu")) and not supports_context(context("cuda"))
    assert not supports_context(context("meta"))


def test_explicit_backends_on_cpu_tensors():
    w = make_workload(0, levels=((4, 4),), batch=1, queries=3, heads=2, channels=8).to("cpu", F32)
    ops = w.operands()
    torch.testing.assert_close(msda(*ops, backend=Backend.EAGER), msda(*ops), rtol=0, atol=0)
    with pytest.raises(NoBackendError):
        msda(*ops, backend=Backend.HIP)
    with pytest.raises(NoBackendError, match="not part of this build"):
        msda(*ops, backend=Backend.TRITON)


# Random shapes, as the GPU sweep draws them (tests/test_hip_msda_hypothesis.py),
# smaller so that the CPU suite stays quick; derandomized, so every run replays the
# same cases.


@st.composite
def cases(draw):
    L = draw(st.integers(1, 4))
    return {
        "levels": tuple((draw(st.integers(1, 24)), draw(st.integers(1, 24))) for _ in range(L)),
        "batch": draw(st.integers(1, 2)),
        "queries": draw(st.integers(1, 40)),
        "heads": draw(st.sampled_from([1, 2, 3, 8])),
        "channels": draw(st.sampled_from([1, 7, 8, 32])),
        "points": draw(st.integers(1, 6)),
        "seed": draw(st.integers(0, 2**31 - 1)),
        "dtype": draw(st.sampled_from([F64, F32, BF16, F16])),
        "softmax": draw(st.booleans()),
        "locations": draw(st.sampled_from(["uniform", "reference"])),
    }


@given(case=cases())
@settings(max_examples=60, deadline=None, derandomize=True, database=None,
          suppress_health_check=[HealthCheck.too_slow, HealthCheck.data_too_large])
def test_random_shapes_match_oracle(case):
    w = make_workload(0, levels=case["levels"], batch=case["batch"], queries=case["queries"], heads=case["heads"],
                      channels=case["channels"], points=case["points"], seed=case["seed"],
                      locations=case["locations"]).to("cpu", case["dtype"])
    check(*w.operands(softmax=case["softmax"]), w.grad_output, softmax=case["softmax"], dtype=case["dtype"],
          label=str(case))
