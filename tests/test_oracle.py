"""Pins the CPU oracle (oracle/msda_oracle.c) before it is trusted as the checker.

Runs on the CPU only. Every function of the oracle (forward, the three gradients,
the softmax method, the float32 pixel map) is checked against something it does
not share code with:

- torch.nn.functional.grid_sample (bilinear, zero padding, align_corners=False)
  at ``2 * loc - 1``, the reference's own definition of the operator
  (backends/reference/msda.py:58-97), and torch autograd through it;
- a torch restatement of the reference eager backend
  (backends/eager/msda_pytorch.py:23-112) and its autograd;
- a brute force written differently: every pixel of every level weighted by the
  tent function max(0, 1 - |x - j|) * max(0, 1 - |y - i|), which is bilinear
  interpolation with zero padding without floor, corners or masks; gradients by
  central differences and by linearity;
- closed forms: 1x1 levels, constant and linear fields, the pixel-boundary table
  with arange values (tests/deformops/test_msda_eager.py:54-80 of the reference),
  one-sided gradients at integer pixels including -1 and the far edge
  (tests/deformops/test_release_regressions.py:264-339), all-out-of-bounds
  (tests/deformops/test_msda_reference.py:132-147), a -inf logit under softmax,
  non-finite locations, empty batches.

``test_checks_detect_planted_mistakes`` shows that a plausible slip (x and y
swapped, a level start off by one, the half-pixel shift dropped, a transposed
channel axis, the softmax skipped) fails the grid_sample comparison.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from oracle.eager import eager_msda, softmax_weights
from oracle.grid_sample_ref import grid_sample_msda
from tests.workloads import CONFIGS, make_workload

F64 = torch.float64


def rel(actual: torch.Tensor, expected: torch.Tensor) -> float:
    actual = actual.to(F64).reshape(expected.shape)
    scale = expected.abs().max().item()
    diff = (actual - expected).abs().max().item()
    return diff if scale == 0.0 else diff / scale


def tables(levels):
    shapes = torch.tensor(levels, dtype=torch.int64).reshape(-1, 2)
    sizes = shapes[:, 0] * shapes[:, 1]
    starts = torch.cat([sizes.new_zeros(1), sizes.cumsum(0)[:-1]])
    return shapes, starts


def random_case(levels, B, Q, H, D, P, *, seed=0, lo=-0.1, hi=1.1):
    g = torch.Generator().manual_seed(seed)
    shapes, starts = tables(levels)
    S, L = int((shapes[:, 0] * shapes[:, 1]).sum()), len(levels)
    value = torch.randn(B, S, H, D, generator=g, dtype=F64)
    loc = torch.rand(B, Q, H, L, P, 2, generator=g, dtype=F64) * (hi - lo) + lo
    logits = torch.randn(B, Q, H, L, P, generator=g, dtype=F64)
    grad = torch.randn(B, Q, H * D, generator=g, dtype=F64)
    return value, shapes, starts, loc, logits, grad


def autograd_grads(fn, value, loc, attn, grad):
    leaves = [t.clone().requires_grad_(True) for t in (value, loc, attn)]
    out = fn(*leaves)
    out.backward(grad)
    return out.detach(), [leaf.grad for leaf in leaves]


SHAPES = [
    pytest.param(((4, 5),), 1, 3, 1, 2, 1, id="one-level"),
    pytest.param(((6, 5), (3, 3), (1, 2)), 2, 7, 3, 4, 3, id="three-levels"),
    pytest.param(((1, 1), (2, 1)), 2, 5, 2, 3, 2, id="degenerate-levels"),
    pytest.param(((8, 8), (4, 4), (2, 2), (1, 1)), 1, 9, 2, 8, 4, id="four-levels"),
]


@pytest.mark.parametrize("softmax", [False, True], ids=["linear", "softmax"])
@pytest.mark.parametrize(("levels", "B", "Q", "H", "D", "P"), SHAPES)
def test_forward_and_gradients_match_grid_sample_autograd(levels, B, Q, H, D, P, softmax):
    value, shapes, starts, loc, logits, grad = random_case(levels, B, Q, H, D, P, seed=len(levels))
    attn = logits if softmax else torch.softmax(logits.flatten(-2), -1).view_as(logits)

    def reference(v, lc, a):
        return grid_sample_msda(v, shapes, lc, softmax_weights(a) if softmax else a)

    ref_out, (ref_gv, ref_gl, ref_ga) = autograd_grads(reference, value, loc, attn, grad)
    out = oracle.forward(value, shapes, starts, loc, attn, softmax=softmax)
    gv, gl, ga = oracle.backward(value, shapes, starts, loc, attn, grad, softmax=softmax)
    assert rel(out, ref_out) < 1e-13
    assert rel(gv, ref_gv) < 1e-13
    assert rel(gl, ref_gl) < 1e-12
    assert rel(ga, ref_ga) < 1e-13


@pytest.mark.parametrize("softmax", [False, True], ids=["linear", "softmax"])
def test_config0_matches_eager_restatement_and_grid_sample(softmax):
    """BASELINE config 0 (the reference's CPU case) at full size, float64."""
    w = make_workload(0)
    value, shapes, starts, loc, attn = w.operands(softmax=softmax)
    attn = attn.view(*attn.shape[:3], shapes.shape[0], -1)

    out = oracle.forward(value, shapes, starts, loc, attn, softmax=softmax)
    gv, gl, ga = oracle.backward(value, shapes, starts, loc, attn, w.grad_output, softmax=softmax)

    def eager(v, lc, a):
        return eager_msda(v, shapes, starts, lc, a, softmax=softmax)

    e_out, (e_gv, e_gl, e_ga) = autograd_grads(eager, value, loc, attn, w.grad_output)
    assert rel(out, e_out) < 1e-13
    assert rel(gv, e_gv) < 1e-13
    assert rel(gl, e_gl) < 1e-12
    assert rel(ga, e_ga) < 1e-13
    weights = softmax_weights(attn) if softmax else attn
    assert rel(out, grid_sample_msda(value, shapes, loc, weights)) < 1e-13


def tent_brute_force(value, shapes, starts, loc, weights):
    """Pure-Python loops over every pixel of every level; tent-function weights."""
    B, S, H, D = value.shape
    _, Q, _, L, P, _ = loc.shape
    out = torch.zeros(B, Q, H, D, dtype=F64)
    for b in range(B):
        for q in range(Q):
            for h in range(H):
                for lvl in range(L):
                    hh, ww = (int(v) for v in shapes[lvl])
                    st = int(starts[lvl])
                    for p in range(P):
                        x = float(loc[b, q, h, lvl, p, 0]) * ww - 0.5
                        y = float(loc[b, q, h, lvl, p, 1]) * hh - 0.5
                        a = float(weights[b, q, h, lvl, p])
                        for i in range(hh):
                            for j in range(ww):
                                t = max(0.0, 1.0 - abs(x - j)) * max(0.0, 1.0 - abs(y - i))
                                if t:
                                    out[b, q, h] += a * t * value[b, st + i * ww + j, h]
    return out.reshape(B, Q, H * D)


def test_forward_matches_tent_brute_force():
    levels = ((3, 4), (2, 2), (1, 3))
    value, shapes, starts, loc, logits, _ = random_case(levels, 2, 4, 2, 3, 2, seed=7, lo=-0.4, hi=1.4)
    weights = torch.softmax(logits.flatten(-2), -1).view_as(logits)
    expected = tent_brute_force(value, shapes, starts, loc, weights)
    assert rel(oracle.forward(value, shapes, starts, loc, weights), expected) < 1e-14


def test_gradients_match_brute_force_linearity_and_central_differences():
    levels = ((3, 4), (2, 3))
    value, shapes, starts, loc, logits, grad = random_case(levels, 1, 3, 2, 3, 2, seed=11, lo=0.05, hi=0.95)
    weights = torch.softmax(logits.flatten(-2), -1).view_as(logits)
    gv, gl, ga = oracle.backward(value, shapes, starts, loc, weights, grad)

    def f(v, lc, a):
        return (tent_brute_force(v, shapes, starts, lc, a) * grad).sum().item()

    # grad_value: the output is linear in value, so grad_value[i] = f(e_i).
    basis_gv = torch.zeros_like(value)
    for idx in range(value.numel()):
        e = torch.zeros(value.numel(), dtype=F64)
        e[idx] = 1.0
        basis_gv.view(-1)[idx] = f(e.view_as(value), loc, weights)
    assert rel(gv, basis_gv) < 1e-14
    # grad_attn: linear in each weight too.
    basis_ga = torch.zeros_like(weights)
    for idx in range(weights.numel()):
        e = torch.zeros(weights.numel(), dtype=F64)
        e[idx] = 1.0
        basis_ga.view(-1)[idx] = f(value, loc, e.view_as(weights))
    assert rel(ga.view_as(weights), basis_ga) < 1e-14
    # grad_loc: central differences (interior, away from pixel boundaries).
    eps = 1e-6
    fd = torch.zeros_like(loc)
    for idx in range(loc.numel()):
        up, dn = loc.clone(), loc.clone()
        up.view(-1)[idx] += eps
        dn.view(-1)[idx] -= eps
        fd.view(-1)[idx] = (f(value, up, weights) - f(value, dn, weights)) / (2 * eps)
    assert rel(gl, fd) < 1e-7


def one_level(h, w, values, xs, ys, *, D=1):
    """Samples (x, y) in pixel coordinates on one h x w level with the given values."""
    shapes, starts = tables(((h, w),))
    value = torch.as_tensor(values, dtype=F64).reshape(1, h * w, 1, 1).expand(1, h * w, 1, D).contiguous()
    n = len(xs)
    loc = torch.zeros(1, n, 1, 1, 1, 2, dtype=F64)
    loc[0, :, 0, 0, 0, 0] = (torch.as_tensor(xs, dtype=F64) + 0.5) / w
    loc[0, :, 0, 0, 0, 1] = (torch.as_tensor(ys, dtype=F64) + 0.5) / h
    attn = torch.ones(1, n, 1, 1, 1, dtype=F64)
    return value, shapes, starts, loc, attn


def test_pixel_boundary_table_with_arange_values():
    """A 1 x 4 level holding 0, 1, 2, 3, sampled along its row."""
    xs = [-1.5, -1.0, -0.5, 0.0, 0.25, 1.0, 2.5, 3.0, 3.5, 4.0, 9.0]
    expected = [0.0, 0.0, 0.0, 0.0, 0.25, 1.0, 2.5, 3.0, 1.5, 0.0, 0.0]
    value, shapes, starts, loc, attn = one_level(1, 4, [0.0, 1.0, 2.0, 3.0], xs, [0.0] * len(xs))
    out = oracle.forward(value, shapes, starts, loc, attn)
    assert out.flatten().tolist() == pytest.approx(expected, abs=1e-15)
    # y = -0.5 halves every value (the row above is zero padding); y = -1 and 1 skip.
    value, shapes, starts, loc, attn = one_level(1, 4, [0.0, 1.0, 2.0, 3.0], [1.0, 1.0, 1.0], [-0.5, -1.0, 1.0])
    assert oracle.forward(value, shapes, starts, loc, attn).flatten().tolist() == pytest.approx([0.5, 0.0, 0.0])


def test_one_by_one_level_closed_form():
    g = torch.Generator().manual_seed(3)
    xs = (torch.rand(20, generator=g, dtype=F64) * 2.4 - 1.2).tolist()
    ys = (torch.rand(20, generator=g, dtype=F64) * 2.4 - 1.2).tolist()
    value, shapes, starts, loc, attn = one_level(1, 1, [2.5], xs, ys, D=3)
    out = oracle.forward(value, shapes, starts, loc, attn).view(20, 3)
    for k, (x, y) in enumerate(zip(xs, ys)):
        inside = -1.0 <= x < 1.0 and -1.0 <= y < 1.0
        expected = 2.5 * (1 - abs(x)) * (1 - abs(y)) if inside else 0.0
        assert out[k].tolist() == pytest.approx([expected] * 3, abs=1e-14)


def test_constant_and_linear_fields_closed_form():
    h, w, D = 5, 7, 2
    g = torch.Generator().manual_seed(5)
    n = 40
    xs = (torch.rand(n, generator=g, dtype=F64) * (w - 1)).tolist()  # interior: all corners in
    ys = (torch.rand(n, generator=g, dtype=F64) * (h - 1)).tolist()
    alpha, beta, gamma = 0.7, -1.3, 0.25
    field = [[alpha * j + beta * i + gamma for j in range(w)] for i in range(h)]
    value, shapes, starts, loc, attn = one_level(h, w, field, xs, ys, D=D)
    attn = torch.rand(attn.shape, generator=g, dtype=F64)
    grad = torch.randn(1, n, D, generator=g, dtype=F64)
    out = oracle.forward(value, shapes, starts, loc, attn).view(n, D)
    _, gl, ga = oracle.backward(value, shapes, starts, loc, attn, grad)
    a = attn.flatten()
    exact = a * (alpha * torch.tensor(xs, dtype=F64) + beta * torch.tensor(ys, dtype=F64) + gamma)
    assert rel(out, exact[:, None].expand(n, D)) < 1e-14
    gsum = grad.view(n, D).sum(-1)
    assert rel(gl.view(n, 2)[:, 0], a * alpha * w * gsum) < 1e-13
    assert rel(gl.view(n, 2)[:, 1], a * beta * h * gsum) < 1e-13
    assert rel(ga.flatten(), (exact[:, None] / a[:, None] * grad.view(n, D)).sum(-1)) < 1e-13
    # A constant field returns weight x in-bounds bilinear mass (1 inside).
    value = torch.full_like(value, 3.0)
    assert rel(oracle.forward(value, shapes, starts, loc, attn).view(n, D), (3.0 * a)[:, None].expand(n, D)) < 1e-14


def test_one_sided_gradient_at_integer_pixels():
    """At an integer pixel the x-gradient is the difference to the right-hand pixel."""
    w = 5
    field = [float(j * j) for j in range(w)]  # v = j^2: right difference 2k + 1
    xs = [-1.0, 0.0, 1.0, 2.0, 3.0, 4.0]
    value, shapes, starts, loc, attn = one_level(1, w, field, xs, [0.0] * len(xs))
    grad = torch.ones(1, len(xs), 1, dtype=F64)
    _, gl, _ = oracle.backward(value, shapes, starts, loc, attn, grad)
    right = [field[0] - 0.0] + [(field[k + 1] if k + 1 < w else 0.0) - field[k] for k in range(w)]
    assert gl.view(-1, 2)[:, 0].tolist() == pytest.approx([w * r for r in right], abs=1e-12)
    # The eager restatement's autograd agrees (same floor convention).
    _, (_, e_gl, _) = autograd_grads(
        lambda v, lc, a: eager_msda(v, shapes, starts, lc, a), value, loc, attn, grad
    )
    assert rel(gl, e_gl) < 1e-14


def test_all_out_of_bounds_gives_zeros():
    value, shapes, starts, loc, logits, grad = random_case(((4, 4), (2, 2)), 2, 5, 2, 3, 2, seed=2)
    loc[..., 0] = torch.where(loc[..., 0] > 0.5, 1.6, -0.6)
    for softmax in (False, True):
        out = oracle.forward(value, shapes, starts, loc, logits, softmax=softmax)
        gv, gl, ga = oracle.backward(value, shapes, starts, loc, logits, grad, softmax=softmax)
        assert out.abs().max() == 0 and gv.abs().max() == 0
        assert gl.abs().max() == 0 and ga.abs().max() == 0


def test_negative_infinite_logit_under_softmax():
    value, shapes, starts, loc, logits, grad = random_case(((4, 4), (2, 2)), 1, 6, 2, 3, 2, seed=9)
    logits[:, :, :, 0, 0] = -math.inf
    out = oracle.forward(value, shapes, starts, loc, logits, softmax=True)
    gv, gl, ga = oracle.backward(value, shapes, starts, loc, logits, grad, softmax=True)
    for t in (out, gv, gl, ga):
        assert torch.isfinite(t).all()
    assert ga.view_as(logits)[:, :, :, 0, 0].abs().max() == 0
    p = softmax_weights(logits)
    assert rel(out, grid_sample_msda(value, shapes, loc, p)) < 1e-13


@pytest.mark.parametrize("bad", [math.inf, -math.inf, math.nan])
def test_nonfinite_locations_are_skipped(bad):
    value, shapes, starts, loc, logits, grad = random_case(((4, 4),), 1, 4, 1, 2, 2, seed=4, lo=0.1, hi=0.9)
    clean = oracle.forward(value, shapes, starts, loc, logits)
    loc2 = loc.clone()
    loc2[0, 1, 0, 0, 1, 0] = bad
    logits2 = logits.clone()
    logits2[0, 1, 0, 0, 1] = 0.0
    out = oracle.forward(value, shapes, starts, loc2, logits2)
    gv, gl, ga = oracle.backward(value, shapes, starts, loc2, logits2, grad)
    assert torch.equal(out[:, [0, 2, 3]], clean[:, [0, 2, 3]])
    for t in (out, gv, gl, ga):
        assert torch.isfinite(t).all()


@pytest.mark.parametrize("axis", ["batch", "queries"])
def test_empty_calls(axis):
    value, shapes, starts, loc, logits, grad = random_case(((3, 3),), 2, 3, 2, 4, 2)
    if axis == "batch":
        value, loc, logits, grad = value[:0], loc[:0], logits[:0], grad[:0]
    else:
        loc, logits, grad = loc[:, :0], logits[:, :0], grad[:, :0]
    out = oracle.forward(value, shapes, starts, loc, logits)
    gv, gl, ga = oracle.backward(value, shapes, starts, loc, logits, grad)
    assert out.shape == (value.shape[0], loc.shape[1], 8)
    assert gv.shape == value.shape and gv.abs().sum() == 0
    assert gl.numel() == 0 and ga.numel() == 0


def test_softmax_method_is_linear_on_normalized_weights_with_jacobian():
    value, shapes, starts, loc, logits, grad = random_case(((5, 4), (2, 3)), 2, 5, 2, 3, 3, seed=13)
    p = softmax_weights(logits)
    assert rel(oracle.forward(value, shapes, starts, loc, logits, softmax=True),
               oracle.forward(value, shapes, starts, loc, p)) < 1e-15
    gv_s, gl_s, ga_s = oracle.backward(value, shapes, starts, loc, logits, grad, softmax=True)
    gv_l, gl_l, ga_l = oracle.backward(value, shapes, starts, loc, p, grad)
    assert rel(gv_s, gv_l) < 1e-15 and rel(gl_s, gl_l) < 1e-15
    # Chain rule through torch.softmax's own autograd.
    lg = logits.clone().requires_grad_(True)
    softmax_weights(lg).backward(ga_l.view_as(logits))
    assert rel(ga_s.view_as(logits), lg.grad) < 1e-13


def test_float32_pixel_map_rounds_like_the_float32_eager_path():
    """With pixel_f32 the oracle lands in the cell float32 arithmetic picks."""
    w = 37
    torch.manual_seed(0)
    # float32 locations next to pixel boundaries whose float32 pixel map
    # floor(fl(fl(x * w) - 0.5)) differs from the exact floor(x * w - 0.5).
    cands = []
    for k in range(1, w):
        x = np.float32((k + 0.5) / w)
        for _ in range(4):
            x = np.nextafter(x, np.float32(-1.0))
        for _ in range(9):
            f32 = np.floor(np.float32(np.float32(x) * np.float32(w)) - np.float32(0.5))
            if float(f32) != math.floor(float(x) * w - 0.5):
                cands.append(float(x))
            x = np.nextafter(x, np.float32(2.0))
    assert cands, "no float32 location rounds across a pixel boundary"
    n = len(cands)
    shapes, starts = tables(((1, w),))
    value = torch.randn(1, w, 1, 2, dtype=torch.float32)
    loc = torch.zeros(1, n, 1, 1, 1, 2, dtype=torch.float32)
    loc[0, :, 0, 0, 0, 0] = torch.tensor(cands, dtype=torch.float32)
    loc[0, :, 0, 0, 0, 1] = 0.5
    attn = torch.ones(1, n, 1, 1, 1, dtype=torch.float32)
    grad = torch.ones(1, n, 2, dtype=torch.float32)

    def eager(v, lc, a):
        return eager_msda(v, shapes, starts, lc, a)

    e_out, (_, e_gl, _) = autograd_grads(eager, value, loc, attn, grad)
    assert rel(oracle.forward(value, shapes, starts, loc, attn), e_out.double()) < 1e-6
    _, gl, _ = oracle.backward(value, shapes, starts, loc, attn, grad)
    assert rel(gl, e_gl.double()) < 1e-5
    # Rounded in float64 instead, the same inputs land in other cells: the output
    # is continuous across a cell edge, the one-sided x-gradient is not.
    _, gl64, _ = oracle.backward(value, shapes, starts, loc, attn, grad, pixel_f32=False)
    assert rel(gl64, e_gl.double()) > 1e-2


MISTAKES = {
    "x-y-swapped": lambda v, sh, st, lc, a: (v, sh, st, lc.flip(-1), a),
    "level-start-off-by-one": lambda v, sh, st, lc, a: (v, sh, st + torch.tensor([0, 1]), lc, a),
    "half-pixel-dropped": lambda v, sh, st, lc, a: (
        v, sh, st, lc + 0.5 / torch.stack([sh[:, 1], sh[:, 0]], -1).to(F64).view(1, 1, 1, -1, 1, 2), a),
    "channels-transposed": lambda v, sh, st, lc, a: (v.flip(-1), sh, st, lc, a),
    "levels-swapped-shapes": lambda v, sh, st, lc, a: (v, sh.flip(-1), st, lc, a),
    "softmax-skipped": lambda v, sh, st, lc, a: (v, sh, st, lc, torch.exp(a)),
}


@pytest.mark.parametrize("mistake", sorted(MISTAKES))
def test_checks_detect_planted_mistakes(mistake):
    """A slip in how the oracle reads its operands fails the grid_sample check."""
    value, shapes, starts, loc, logits, _ = random_case(((5, 6), (3, 2)), 1, 6, 2, 3, 2, seed=21)
    p = softmax_weights(logits)
    expected = grid_sample_msda(value, shapes, loc, p)
    assert rel(oracle.forward(value, shapes, starts, loc, p), expected) < 1e-13
    planted = oracle.forward(*MISTAKES[mistake](value, shapes, starts, loc, p))
    assert rel(planted, expected) > 1e-3, f"planted mistake {mistake} went unnoticed"


def test_workload_generators_are_seeded_and_shaped():
    for idx, cfg in CONFIGS.items():
        if idx == 4:
            w = make_workload(idx, batch=1, queries=64)
        else:
            w = make_workload(idx, batch=1, queries=min(64, cfg.queries or 64))
        B, S, H, D, Q, L, P = w.sizes
        assert (H, D, P) == (8, 32, 4) and L == len(cfg.levels)
        assert S == sum(h * ww for h, ww in cfg.levels)
        again = make_workload(idx, batch=1, queries=Q)
        assert torch.equal(w.value, again.value) and torch.equal(w.sampling_locations, again.sampling_locations)
        assert torch.allclose(w.attention_weights.sum(-1), torch.ones((), dtype=F64), atol=1e-12)
