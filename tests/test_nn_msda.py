"""The MultiScaleDeformAttn2d layer (reference ``nn/msda.py``; its tests
``tests/deformops/test_msda_state_dict.py`` and
``tests/deformops/test_msda_gradcheck.py:116-156`` are the model here).

CPU: construction checks, Deformable DETR's initialization, the state-dict upgrade
and the sampling-location math. GPU: the layer on the HIP kernels against the same
layer in float64 on the CPU with the torch restatement of the eager algorithm
(``oracle.eager``) as its backend, outputs and every gradient; and a float64
gradcheck through the HIP backward.
"""

from __future__ import annotations

import copy
import math

import pytest
import torch

from deformops_amd.core.errors import NoBackendError
from deformops_amd.core.runtime import Method
from deformops_amd.nn import MultiScaleDeformAttn2d
from deformops_amd.registry import Backend, MSDABackend
from oracle.eager import eager_msda

F32, F64, BF16 = torch.float32, torch.float64, torch.bfloat16


class EagerOracleBackend:
    """An ``MSDABackend`` adapter over the CPU oracle (test infrastructure).

    With ``locations`` set, it samples there instead (same values, gradients passed
    straight through to the layer's own locations).
    """

    name = "eager-oracle"

    def __init__(self) -> None:
        self.locations: torch.Tensor | None = None

    def supports(self, context) -> bool:  # noqa: ANN001
        return True

    def forward(self, value, spatial_shapes, level_start_index, loc, weights, chunk_step, method):  # noqa: ANN001, ANN201, PLR0913
        if self.locations is not None:
            loc = loc + (self.locations.to(loc) - loc).detach()
        return eager_msda(value, spatial_shapes, level_start_index, loc, weights,
                          softmax=Method(method) is Method.SOFTMAX)


def rel_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    actual = actual.detach().to("cpu", F64)
    expected = expected.detach().to("cpu", F64)
    scale = expected.abs().max().item()
    diff = (actual - expected).abs().max().item()
    return diff / scale if scale else diff


def pyramid(levels):
    shapes = torch.tensor(levels, dtype=torch.int64)
    sizes = shapes[:, 0] * shapes[:, 1]
    starts = torch.cat([sizes.new_zeros(1), sizes.cumsum(0)[:-1]])
    return shapes, starts, int(sizes.sum())


# Construction and parameters (CPU).


def test_adapter_is_a_backend():
    assert isinstance(EagerOracleBackend(), MSDABackend)


@pytest.mark.parametrize(
    ("kwargs", "fragment"),
    [
        ({"dim": 48, "num_heads": 2}, "power of 2"),  # 24 channels per head
        ({"dim": 30, "num_heads": 4}, "divisible"),
        ({"dim": 32, "num_heads": 0}, "num_heads"),
        ({"dim": 32, "num_heads": 2, "num_levels": 0}, "num_levels"),
        ({"dim": 32, "num_heads": 2, "num_points": -1}, "num_points"),
    ],
)
def test_invalid_sizes_raise(kwargs, fragment):
    args = {"num_levels": 2, **kwargs}
    with pytest.raises(ValueError, match=fragment):
        MultiScaleDeformAttn2d(**args)


def test_initialization_is_deformable_detr():
    H, L, P = 8, 3, 4
    m = MultiScaleDeformAttn2d(dim=64, num_heads=H, num_levels=L, num_points=P)
    bias = m.proj_offset.bias.detach().view(H, L, P, 2)
    for h in range(H):
        a = 2.0 * math.pi * h / H
        c, s = math.cos(a), math.sin(a)
        top = max(abs(c), abs(s))
        for k in range(P):
            want = torch.tensor([c / top * (k + 1), s / top * (k + 1)])
            for lvl in range(L):
                torch.testing.assert_close(bias[h, lvl, k], want, atol=1e-5, rtol=0)  # float32 angles
    # The first head looks along +x with points at 1, 2, ... pixels.
    assert torch.equal(bias[0, :, :, 1], torch.zeros(L, P))
    assert torch.count_nonzero(m.proj_offset.weight) == 0
    assert torch.count_nonzero(m.proj_weights.weight) == 0
    assert torch.count_nonzero(m.proj_weights.bias) == 0
    assert torch.count_nonzero(m.proj_value.bias) == 0 and torch.count_nonzero(m.proj_output.bias) == 0
    assert m.method is Method.SOFTMAX
    assert MultiScaleDeformAttn2d(dim=32, num_heads=2, num_levels=1, method="linear").method is Method.LINEAR


def test_widths():
    m = MultiScaleDeformAttn2d(dim=32, dim_value=24, dim_output=40, num_heads=4, num_levels=2, num_points=3)
    assert m.proj_value.in_features == 24 and m.proj_output.out_features == 40
    assert m.proj_offset.out_features == 4 * 2 * 3 * 2 and m.proj_weights.out_features == 4 * 2 * 3


# The state-dict upgrade (reference tests/deformops/test_msda_state_dict.py).


def small_layer():
    return MultiScaleDeformAttn2d(dim=16, num_heads=2, num_levels=1, num_points=1)


def test_legacy_names_load():
    m = small_layer()
    legacy = {
        "sampling_offsets.weight": torch.full_like(m.proj_offset.weight, 1.0),
        "sampling_offsets.bias": torch.full_like(m.proj_offset.bias, 2.0),
        "attention_weights.weight": torch.full_like(m.proj_weights.weight, 3.0),
        "attention_weights.bias": torch.full_like(m.proj_weights.bias, 4.0),
        "value_proj.weight": torch.full_like(m.proj_value.weight, 5.0),
        "value_proj.bias": torch.full_like(m.proj_value.bias, 6.0),
        "output_proj.weight": torch.full_like(m.proj_output.weight, 7.0),
        "output_proj.bias": torch.full_like(m.proj_output.bias, 8.0),
    }
    result = m.load_state_dict(legacy, strict=True)
    assert not result.missing_keys and not result.unexpected_keys
    assert torch.all(m.proj_offset.bias == 2.0) and torch.all(m.proj_output.weight == 7.0)


def test_unknown_key_reported_when_strict():
    m = small_layer()
    state = {**m.state_dict(), "unknown_legacy_thing.weight": torch.zeros(1)}
    with pytest.raises(RuntimeError, match="unknown_legacy_thing"):
        m.load_state_dict(state, strict=True)


def test_unknown_key_ignored_when_not_strict():
    m = small_layer()
    state = {
        "sampling_offsets.weight": torch.ones_like(m.proj_offset.weight),
        "sampling_offsets.bias": torch.ones_like(m.proj_offset.bias),
        "unknown_legacy_thing.weight": torch.zeros(1),
    }
    result = m.load_state_dict(state, strict=False)
    assert "unknown_legacy_thing.weight" in result.unexpected_keys
    assert torch.equal(m.proj_offset.weight, torch.ones_like(m.proj_offset.weight))


def test_current_state_dict_round_trips():
    a, b = small_layer(), small_layer()
    torch.nn.init.normal_(a.proj_offset.weight)
    b.load_state_dict(a.state_dict(), strict=True)
    assert torch.equal(a.proj_offset.weight, b.proj_offset.weight)


# The sampling places (CPU).


def test_sampling_locations_points_and_boxes():
    torch.manual_seed(3)
    B, Q, H, L, P = 2, 5, 2, 2, 3
    m = MultiScaleDeformAttn2d(dim=8, num_heads=H, num_levels=L, num_points=P).double()
    torch.nn.init.normal_(m.proj_offset.weight)
    shapes = torch.tensor([[6, 10], [3, 5]])
    q = torch.randn(B, Q, 8, dtype=F64)
    off = m.proj_offset(q).view(B, Q, H, L, P, 2)
    points = torch.rand(B, Q, L, 2, dtype=F64)
    loc = m.sampling_locations(q, points, shapes)
    boxes = torch.rand(B, Q, L, 4, dtype=F64)
    loc_box = m.sampling_locations(q, boxes, shapes)
    for b in range(B):
        for i in range(Q):
            for h in range(H):
                for lvl in range(L):
                    height, width = shapes[lvl].tolist()
                    for k in range(P):
                        dx, dy = off[b, i, h, lvl, k].tolist()
                        x, y = points[b, i, lvl].tolist()
                        assert loc[b, i, h, lvl, k].tolist() == pytest.approx([x + dx / width, y + dy / height])
                        cx, cy, w, hh = boxes[b, i, lvl].tolist()
                        assert loc_box[b, i, h, lvl, k].tolist() == pytest.approx(
                            [cx + dx / P * w / 2, cy + dy / P * hh / 2])
    with pytest.raises(ValueError, match="reference points"):
        m.sampling_locations(q, torch.rand(B, Q, L, 3, dtype=F64), shapes)


def test_cpu_layer_runs_the_eager_backend():
    """Without a backend the layer's CPU call runs Backend.EAGER; it matches the same
    layer over the oracle adapter, output and gradients; asking for HIP raises."""
    torch.manual_seed(0)
    m = MultiScaleDeformAttn2d(dim=16, num_heads=2, num_levels=2, num_points=4).to(F64)
    shapes, starts, n = pyramid([[4, 4], [2, 2]])
    g = torch.Generator().manual_seed(1)
    q, ref, x = (torch.randn(1, 3, 16, generator=g, dtype=F64), torch.rand(1, 3, 2, 2, generator=g, dtype=F64),
                 torch.randn(1, n, 16, generator=g, dtype=F64))
    oracle_layer = copy.deepcopy(m)
    oracle_layer.backend = EagerOracleBackend()
    out = m(q, ref, x, shapes, starts)
    want = oracle_layer(q, ref, x, shapes, starts)
    assert rel_err(out, want) <= 1e-12
    out.sum().backward()
    want.sum().backward()
    for (name, p), p_ref in zip(m.named_parameters(), oracle_layer.parameters(), strict=True):
        assert rel_err(p.grad, p_ref.grad) <= 1e-10, name
    m.backend = Backend.HIP
    with pytest.raises(NoBackendError):
        m(q, ref, x, shapes, starts)


def test_cpu_layer_with_the_oracle_backend():
    """The layer's own code path around an adapter: the output of a layer whose
    offsets and weights are zero is the bilinear sample of the projected values at
    the reference point, averaged over the heads' uniform softmax weights."""
    m = MultiScaleDeformAttn2d(dim=8, num_heads=1, num_levels=1, num_points=2, backend=EagerOracleBackend()).double()
    with torch.no_grad():
        m.proj_offset.bias.zero_()
        m.proj_value.weight.copy_(torch.eye(8, dtype=F64))
        m.proj_output.weight.copy_(torch.eye(8, dtype=F64))
    shapes, starts, n = pyramid([[2, 2]])
    v = torch.randn(1, n, 8, dtype=F64)
    # The centre of a 2 x 2 map averages all four positions.
    out = m(torch.randn(1, 1, 8, dtype=F64), torch.full((1, 1, 1, 2), 0.5, dtype=F64), v, shapes, starts)
    torch.testing.assert_close(out[0, 0], v[0].mean(0))


# The layer on the HIP kernels (GPU).


def make_pair(device, dtype, method, *, boxes=False):
    torch.manual_seed(11)
    levels = [[16, 16], [8, 8], [4, 4]]
    B, Q, dim, H, P = 2, 40, 64, 2, 4
    m = MultiScaleDeformAttn2d(dim=dim, dim_value=48, num_heads=H, num_levels=len(levels), num_points=P,
                               method=method)
    with torch.no_grad():  # offsets and weights that depend on the query
        m.proj_offset.weight.normal_(0.0, 0.05)
        m.proj_weights.weight.normal_(0.0, 0.2)
        m.proj_weights.bias.normal_(0.0, 0.2)
    ref = copy.deepcopy(m).double()
    ref.backend = EagerOracleBackend()
    shapes, starts, n = pyramid(levels)
    q = torch.randn(B, Q, dim, dtype=F64)
    p = torch.rand(B, Q, len(levels), 4 if boxes else 2, dtype=F64) * 0.8 + 0.1
    if boxes:
        p[..., 2:] = p[..., 2:] * 0.4
    v = torch.randn(B, n, 48, dtype=F64)
    return m.to(device, dtype), ref, (q, p, v, shapes, starts)


def run_layer(m, q, p, v, shapes, starts, grad, *, mask=None):
    leaves = [t.clone().requires_grad_(True) for t in (q, p, v)]
    out = m(*leaves, shapes, starts, mask)
    out.backward(grad)
    grads = [t.grad for t in leaves] + [prm.grad for prm in m.parameters()]
    return out, grads


TOL = {F32: 2e-4, BF16: 2e-2}


@pytest.mark.gpu
@pytest.mark.parametrize("boxes", [False, True], ids=["points", "boxes"])
@pytest.mark.parametrize("method", ["softmax", "linear"])
@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_layer_matches_float64_oracle_layer(device, dtype, method, boxes):
    m, ref, (q, p, v, shapes, starts) = make_pair(device, dtype, method, boxes=boxes)
    grad = torch.randn(q.shape[0], q.shape[1], 64, dtype=F64)
    mask = torch.zeros(v.shape[0], v.shape[1], dtype=torch.bool)
    mask[1, -20:] = True  # padded tokens of the second image
    cast = lambda t: t.to(device, dtype)  # noqa: E731
    # The layer computes its sampling locations in its own dtype. bf16 puts them on a
    # 1/16-pixel grid at 16 x 16: the bilinear weights move by up to 0.03, and a
    # coordinate on a pixel boundary has a one-sided gradient. So the reference
    # samples where the layer sampled.
    own = m.sampling_locations
    seen = {}
    m.sampling_locations = lambda *a: seen.setdefault("loc", own(*a))
    out, grads = run_layer(m, cast(q), cast(p), cast(v), shapes.to(device), starts.to(device), cast(grad),
                           mask=mask.to(device))
    ref.backend.locations = seen["loc"].detach().to("cpu", F64)
    # The float64 reference layer sees the same rounded inputs.
    rq, rp, rv = (cast(t).to("cpu", F64) for t in (q, p, v))
    ref_out, ref_grads = run_layer(ref, rq, rp, rv, shapes, starts, cast(grad).to("cpu", F64), mask=mask)
    tol = TOL[dtype]
    assert rel_err(out, ref_out) <= tol
    names = ["q", "p", "v"] + [n for n, _ in m.named_parameters()]
    errs = {n: rel_err(g, rg) for n, g, rg in zip(names, grads, ref_grads)}
    assert all(e <= tol for e in errs.values()), sorted(errs.items())


@pytest.mark.gpu
@pytest.mark.parametrize("method", ["linear", "softmax"])
def test_layer_gradcheck_float64(device, method):
    """Reference tests/deformops/test_msda_gradcheck.py:116-156 on the HIP kernels."""
    torch.manual_seed(0)
    B, Q, dim, H, W = 1, 2, 16, 16, 16
    m = MultiScaleDeformAttn2d(dim=dim, num_heads=1, num_levels=1, num_points=4, method=method).to(device, F64)
    torch.nn.init.zeros_(m.proj_offset.bias)
    torch.nn.init.normal_(m.proj_weights.weight, std=0.01)
    torch.nn.init.normal_(m.proj_weights.bias, std=0.01)
    q = torch.randn(B, Q, dim, device=device, dtype=F64, requires_grad=True)
    p = (torch.rand(B, Q, 1, 2, device=device, dtype=F64) * 0.5 + 0.25).requires_grad_(True)
    v = torch.randn(B, H * W, dim, device=device, dtype=F64, requires_grad=True)
    shapes = torch.tensor([[H, W]], device=device)
    starts = torch.tensor([0], device=device)
    # grad_value sums its contributions in an order that may differ between runs.
    assert torch.autograd.gradcheck(lambda a, b, c: m(a, b, c, shapes, starts), (q, p, v), nondet_tol=1e-10)
