"""The committed golden vectors (tests/golden/*.pt): the oracle and the HIP path.

Each fixture holds inputs in the dtype they run in and the float64 oracle's
forward and gradients for both methods (written by tests/golden/make_golden.py,
which checks them against grid_sample autograd first). On the CPU the oracle must
reproduce them (a change to the oracle shows up here); on the GPU the HIP path
through ``deformops_amd.registry.msda`` must match them within the north-star
tolerances.
"""

from __future__ import annotations

from pathlib import Path

import pytest
import torch

import oracle
from oracle.eager import softmax_weights
from oracle.grid_sample_ref import grid_sample_msda

GOLDEN = sorted((Path(__file__).resolve().parent / "golden").glob("*.pt"))
F64 = torch.float64
KEYS = ("output", "grad_value", "grad_loc", "grad_attn")
TOL = {torch.float64: (1e-10, 1e-10), torch.float32: (1e-5, 1e-4), torch.bfloat16: (2e-2, 2e-2),
       torch.float16: (2e-2, 2e-2)}


def rel(actual, expected):
    actual = actual.detach().to("cpu", F64).reshape(expected.shape)
    expected = expected.to(F64)
    scale = expected.abs().max().item()
    diff = (actual - expected).abs().max().item()
    return diff if scale == 0.0 else diff / scale


def load(path):
    return torch.load(path, weights_only=True)


def operands(fx, softmax):
    return (fx["value"], fx["spatial_shapes"], fx["level_start_index"], fx["sampling_locations"],
            fx["logits"] if softmax else fx["weights"])


def test_fixtures_exist():
    names = {p.stem for p in GOLDEN}
    assert {"tiny_f64", "boundary_f32", "config0_slice_f32", "headline_small_bf16"} <= names


@pytest.mark.parametrize("softmax", [False, True], ids=["linear", "softmax"])
@pytest.mark.parametrize("path", GOLDEN, ids=[p.stem for p in GOLDEN])
def test_oracle_reproduces_golden(path, softmax):
    fx = load(path)
    tag = "softmax" if softmax else "linear"
    pixel_f32 = fx["value"].dtype != F64
    ops = operands(fx, softmax)
    out = oracle.forward(*ops, softmax=softmax, pixel_f32=pixel_f32)
    gv, gl, ga = oracle.backward(*ops, fx["grad_output"], softmax=softmax, pixel_f32=pixel_f32)
    tol = 1e-13 if fx["value"].dtype == F64 else 1e-6  # expected values stored in float32
    for key, got in zip(KEYS, (out, gv, gl, ga)):
        assert rel(got, fx[f"{tag}.{key}"]) < tol, key


@pytest.mark.parametrize("path", GOLDEN, ids=[p.stem for p in GOLDEN])
def test_golden_forward_matches_grid_sample(path):
    fx = load(path)
    v, sh, _, lc, _ = operands(fx, False)
    expected = grid_sample_msda(v.to(F64), sh, lc.to(F64), fx["weights"].to(F64))
    assert rel(fx["linear.output"], expected) < 1e-5
    expected = grid_sample_msda(v.to(F64), sh, lc.to(F64), softmax_weights(fx["logits"].to(F64)))
    assert rel(fx["softmax.output"], expected) < 1e-5


def test_boundary_fixture_holds_the_table():
    fx = load(next(p for p in GOLDEN if p.stem == "boundary_f32"))
    row = fx["linear.output"][0, :, 0].tolist()
    assert row == pytest.approx([0.0, 0.0, 0.0, 0.0, 0.25, 1.0, 2.5, 3.0, 1.5, 0.0, 0.0], abs=1e-7)


@pytest.mark.gpu
@pytest.mark.parametrize("softmax", [False, True], ids=["linear", "softmax"])
@pytest.mark.parametrize("path", GOLDEN, ids=[p.stem for p in GOLDEN])
def test_hip_matches_golden(device, path, softmax):
    from deformops_amd.registry import msda  # noqa: PLC0415

    fx = load(path)
    tag = "softmax" if softmax else "linear"
    dtype = fx["value"].dtype
    v, sh, st, lc, at = (t.to(device) for t in operands(fx, softmax))
    leaves = [t.clone().requires_grad_(True) for t in (v, lc, at)]
    out = msda(leaves[0], sh, st, leaves[1], leaves[2], method="softmax" if softmax else "linear")
    out.backward(fx["grad_output"].to(device))
    torch.cuda.synchronize()
    fwd_tol, bwd_tol = TOL[dtype]
    got = (out, leaves[0].grad, leaves[1].grad, leaves[2].grad)
    errs = {k: rel(g, fx[f"{tag}.{k}"]) for k, g in zip(KEYS, got)}
    tols = {"output": fwd_tol, "grad_value": bwd_tol, "grad_loc": bwd_tol, "grad_attn": bwd_tol}
    assert all(errs[k] <= tols[k] for k in KEYS), f"{path.stem} {tag}: {errs} vs {tols}"
