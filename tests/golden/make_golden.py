"""Writes the golden MSDA vectors under tests/golden/ (inputs and expected outputs).

The reference holds no fixture files for this path (its parity tests draw seeded
inputs and compare against its eager and grid_sample backends), so the vectors are
made here: the float64 C oracle computes the forward and the three gradients, and
every case is checked against torch's grid_sample definition of the operator and
its autograd (the reference's backends/reference/msda.py:58-97) before it is
written. Each file is a dict of tensors, loadable with
``torch.load(path, weights_only=True)``.

    python -m tests.golden.make_golden
"""

from __future__ import annotations

from pathlib import Path

import torch

import oracle
from oracle.eager import softmax_weights
from oracle.grid_sample_ref import grid_sample_msda
from tests.workloads import make_workload

GOLDEN_DIR = Path(__file__).resolve().parent
F64 = torch.float64


def _tables(levels):
    shapes = torch.tensor(levels, dtype=torch.int64).reshape(-1, 2)
    sizes = shapes[:, 0] * shapes[:, 1]
    return shapes, torch.cat([sizes.new_zeros(1), sizes.cumsum(0)[:-1]])


def _tiny():
    g = torch.Generator().manual_seed(101)
    shapes, starts = _tables(((3, 4), (2, 2), (1, 3)))
    S = int((shapes[:, 0] * shapes[:, 1]).sum())
    B, Q, H, D, L, P = 2, 5, 2, 8, 3, 2
    return {
        "value": torch.randn(B, S, H, D, generator=g, dtype=F64),
        "spatial_shapes": shapes,
        "level_start_index": starts,
        "sampling_locations": torch.rand(B, Q, H, L, P, 2, generator=g, dtype=F64) * 1.4 - 0.2,
        "logits": torch.randn(B, Q, H, L, P, generator=g, dtype=F64),
        "grad_output": torch.randn(B, Q, H * D, generator=g, dtype=F64),
    }


def _boundary():
    """The pixel-boundary table: a 1 x 4 level holding 0..3 (times 1, 2 per channel)."""
    shapes, starts = _tables(((1, 4),))
    xs = torch.tensor([-1.5, -1.0, -0.5, 0.0, 0.25, 1.0, 2.5, 3.0, 3.5, 4.0, 9.0], dtype=F64)
    n = xs.numel()
    value = torch.arange(4, dtype=F64).view(1, 4, 1, 1) * torch.tensor([1.0, 2.0], dtype=F64).view(1, 1, 1, 2)
    loc = torch.zeros(1, n, 1, 1, 1, 2, dtype=F64)
    loc[0, :, 0, 0, 0, 0] = (xs + 0.5) / 4
    loc[0, :, 0, 0, 0, 1] = 0.5
    return {
        "value": value.repeat(1, 1, 1, 4),  # D = 8
        "spatial_shapes": shapes,
        "level_start_index": starts,
        "sampling_locations": loc,
        "logits": torch.zeros(1, n, 1, 1, 1, dtype=F64),
        "grad_output": torch.ones(1, n, 8, dtype=F64),
    }


def _config(idx, **resize):
    w = make_workload(idx, **resize)
    shapes = w.spatial_shapes
    return {
        "value": w.value,
        "spatial_shapes": shapes,
        "level_start_index": w.level_start_index,
        "sampling_locations": w.sampling_locations,
        "logits": w.logits.view(*w.logits.shape[:3], shapes.shape[0], -1),
        "grad_output": w.grad_output,
    }


# name -> (inputs, dtype the inputs are stored and run in)
CASES = {
    "tiny_f64": (_tiny, F64),
    "boundary_f32": (_boundary, torch.float32),
    "config0_slice_f32": (lambda: _config(0, heads=1, channels=8, queries=96), torch.float32),
    "headline_small_bf16": (
        lambda: _config(4, batch=1, heads=2, channels=16, queries=96, levels=((16, 16), (8, 8), (4, 4))),
        torch.bfloat16,
    ),
}


def _expected(inputs, softmax, pixel_f32):
    args = (inputs["value"], inputs["spatial_shapes"], inputs["level_start_index"], inputs["sampling_locations"])
    attn = inputs["logits"] if softmax else inputs["weights"]
    out = oracle.forward(*args, attn, softmax=softmax, pixel_f32=pixel_f32)
    gv, gl, ga = oracle.backward(*args, attn, inputs["grad_output"], softmax=softmax, pixel_f32=pixel_f32)
    return out, gv, gl, ga.view_as(attn)


def _cross_check(inputs, softmax, expected):
    """The oracle's vectors against grid_sample and its autograd, float64."""
    attn_key = "logits" if softmax else "weights"
    leaves = [inputs[k].clone().requires_grad_(True) for k in ("value", "sampling_locations", attn_key)]
    weights = softmax_weights(leaves[2]) if softmax else leaves[2]
    out = grid_sample_msda(leaves[0], inputs["spatial_shapes"], leaves[1], weights)
    out.backward(inputs["grad_output"])
    got = (out.detach(), leaves[0].grad, leaves[1].grad, leaves[2].grad)
    for name, a, b in zip(("output", "grad_value", "grad_loc", "grad_attn"), expected, got):
        scale = max(b.abs().max().item(), 1e-300)
        err = (a - b).abs().max().item() / scale
        if not err < 1e-12:
            raise AssertionError(f"oracle {name} disagrees with grid_sample autograd: {err:.3g}")


def make() -> list[Path]:
    written = []
    for name, (build, store) in CASES.items():
        inputs = build()
        inputs["weights"] = softmax_weights(inputs["logits"])  # the linear method's operand
        # Round the inputs to the storage dtype first; the oracle runs on the rounded values.
        rounded = {
            k: (v.to(store).to(F64) if v.is_floating_point() else v) for k, v in inputs.items()
        }
        record = {k: (v.to(store) if v.is_floating_point() else v) for k, v in inputs.items()}
        for softmax in (False, True):
            _cross_check(rounded, softmax, _expected(rounded, softmax, pixel_f32=False))
            # Stored: the pixel map rounded in float32 for every dtype but float64, as
            # the kernels and the reference's eager path round it.
            expected = _expected(rounded, softmax, pixel_f32=store != F64)
            tag = "softmax" if softmax else "linear"
            for key, t in zip(("output", "grad_value", "grad_loc", "grad_attn"), expected):
                record[f"{tag}.{key}"] = t if store == F64 else t.to(torch.float32)
        path = GOLDEN_DIR / f"{name}.pt"
        torch.save(record, path)
        written.append(path)
    return written


if __name__ == "__main__":
    for p in make():
        print(p, p.stat().st_size)
