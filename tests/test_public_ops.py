"""The public operators ``torch.ops.deformops.msda`` / ``msda_softmax`` under
torch's function transforms: schema, fake tensors, ``torch.compile`` (fullgraph and
dynamic), ``torch.export`` and ``torch.library.opcheck`` (reference
``tests/deformops/test_public_ops.py:755-900``, whose checks run here on the HIP
kernels instead of the eager CPU backend).
"""

from __future__ import annotations

from collections.abc import Callable
from typing import Any

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import deformops_amd.registry  # noqa: F401  (defines the operators)
from deformops_amd.registry import msda

F32 = torch.float32
SCHEMA = (
    "(Tensor value, Tensor spatial_shapes, Tensor level_start_index, "
    "Tensor sampling_locations, Tensor attention_weights) -> Tensor"
)
CASES = [("msda", "linear"), ("msda_softmax", "softmax")]


def qualified(name: str) -> str:
    return f"deformops::{name}"


def op_of(name: str):
    return getattr(torch.ops.deformops, name)


def make_operands(device, batch: int, size: int, requires_grad: bool) -> tuple[torch.Tensor, ...]:
    """Two levels of ``size`` x ``size + 1`` and half that; 6 queries, 2 heads of 8."""
    g = torch.Generator().manual_seed(batch * 100 + size)
    levels = [(size, size + 1), (size // 2 + 1, size // 2 + 2)]
    shapes = torch.tensor(levels, dtype=torch.int64)
    areas = shapes[:, 0] * shapes[:, 1]
    starts = torch.cat([areas.new_zeros(1), areas.cumsum(0)[:-1]])
    S, Q, H, D, L, P = int(areas.sum()), 6, 2, 8, len(levels), 3
    value = torch.randn(batch, S, H, D, generator=g)
    loc = torch.rand(batch, Q, H, L, P, 2, generator=g) * 0.9 + 0.05
    attn = torch.rand(batch, Q, H, L * P, generator=g)
    out = [value.to(device), shapes.to(device), starts.to(device), loc.to(device), attn.to(device)]
    for i in (0, 3, 4):
        out[i].requires_grad_(requires_grad)
    return tuple(out)


def detached(operands, requires_grad: bool):
    return tuple(t.detach().clone().requires_grad_(requires_grad) if t.is_floating_point() else t
                 for t in operands)


def graph_op_names(gm: torch.fx.GraphModule) -> set[str]:
    """Qualified names (``ns::op``) of the operators a graph calls."""
    names = set()
    for node in gm.graph.nodes:
        if node.op != "call_function":
            continue
        target = node.target
        if isinstance(target, torch._ops.OpOverloadPacket):
            names.add(target._qualified_op_name)
        elif isinstance(target, torch._ops.OpOverload):
            names.add(target._schema.name)
    return names


@pytest.mark.parametrize(("name", "method"), CASES)
def test_schema(name, method):
    assert str(op_of(name).default._schema) == f"{qualified(name)}{SCHEMA}"


@pytest.mark.gpu
@pytest.mark.parametrize(("name", "method"), CASES)
def test_op_and_registry_agree(device, name, method):
    operands = make_operands(device, 2, 5, True)
    through_op, through_registry = detached(operands, True), detached(operands, True)
    outs = [op_of(name)(*through_op), msda(*through_registry, method=method)]
    grad = torch.randn_like(outs[0])
    for o in outs:
        o.backward(grad)
    torch.testing.assert_close(outs[0], outs[1], rtol=0, atol=0)
    for a, b in zip(through_op, through_registry):
        if a.grad is not None:
            # grad_value sums each element's contributions in an order that may vary.
            torch.testing.assert_close(a.grad, b.grad)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [torch.no_grad, torch.inference_mode])
@pytest.mark.parametrize(("name", "method"), CASES)
def test_runs_without_autograd(device, name, method, mode: Callable[[], Any]):
    operands = make_operands(device, 2, 5, True)
    expected = msda(*detached(operands, False), method=method)
    with mode():
        out = op_of(name)(*operands)
    assert not out.requires_grad
    torch.testing.assert_close(out, expected, rtol=0, atol=0)


@pytest.mark.gpu
@pytest.mark.parametrize(("name", "method"), CASES)
def test_runs_under_fake_tensor_mode(device, name, method):
    operands = make_operands(device, 2, 5, True)
    expected = op_of(name)(*operands)
    with FakeTensorMode() as mode:
        out = op_of(name)(*(mode.from_tensor(t) for t in operands))
    assert out.shape == expected.shape and out.dtype == expected.dtype


@pytest.mark.gpu
@pytest.mark.parametrize(("name", "method"), CASES)
def test_compile_records_the_public_op_and_aot_the_private_ops(device, name, method):
    from functorch.compile import make_boxed_func  # noqa: PLC0415
    from torch._dynamo.backends.common import aot_autograd  # noqa: PLC0415

    dynamo_names: set[str] = set()
    aot_names: dict[str, set[str]] = {"forward": set(), "backward": set()}

    def recorder(kind: str):
        def compiler(gm: torch.fx.GraphModule, _inputs: Any):
            aot_names[kind] |= graph_op_names(gm)
            return make_boxed_func(gm.forward)

        return compiler

    aot_backend = aot_autograd(fw_compiler=recorder("forward"), bw_compiler=recorder("backward"))

    def backend(gm: torch.fx.GraphModule, inputs: Any):
        dynamo_names.update(graph_op_names(gm))
        return aot_backend(gm, inputs)

    torch._dynamo.reset()
    compiled = torch.compile(lambda *a: msda(*a, method=method), backend=backend, fullgraph=True)
    operands = make_operands(device, 2, 5, True)
    out = compiled(*operands)
    out.sum().backward()
    assert qualified(name) in dynamo_names
    prefix = "deformops_hip::msda_softmax" if method == "softmax" else "deformops_hip::msda"
    assert f"{prefix}_forward" in aot_names["forward"]
    assert f"{prefix}_backward" in aot_names["backward"]
    for kind, names in aot_names.items():
        assert qualified(name) not in names, kind
    torch.testing.assert_close(out, msda(*detached(operands, False), method=method), rtol=0, atol=0)


@pytest.mark.gpu
@pytest.mark.parametrize(("name", "method"), CASES)
def test_dynamic_compile_across_batch_and_size(device, name, method):
    torch._dynamo.reset()
    compiled = torch.compile(lambda *a: msda(*a, method=method), backend="aot_eager", dynamic=True,
                             fullgraph=True)
    for batch, size in ((2, 5), (3, 7)):
        operands = make_operands(device, batch, size, True)
        out = compiled(*operands)
        out.sum().backward()
        torch.testing.assert_close(out, msda(*detached(operands, False), method=method), rtol=0, atol=0)


@pytest.mark.gpu
@pytest.mark.parametrize(("name", "method"), CASES)
def test_export_keeps_the_public_op_until_decomposed(device, name, method):
    class Wrapper(torch.nn.Module):
        def forward(self, *operands):
            return op_of(name)(*operands)

    operands = make_operands(device, 2, 5, False)
    exported = torch.export.export(Wrapper(), operands)
    assert qualified(name) in graph_op_names(exported.graph_module)
    decomposed = exported.run_decompositions()
    assert qualified(name) not in graph_op_names(decomposed.graph_module)
    torch.testing.assert_close(decomposed.module()(*operands), op_of(name)(*operands), rtol=0, atol=0)


@pytest.mark.gpu
@pytest.mark.parametrize(("name", "method"), CASES)
def test_opcheck(device, name, method):
    torch.library.opcheck(op_of(name).default, make_operands(device, 2, 5, True))


# vmap: the mapped axis folds into the batch axis (reference
# registry/_vmap.py:19-82); the level tables may not be mapped.


def test_vmap_over_level_tables_raises():
    """Refused by the vmap rule itself, before any backend runs (so on the CPU too)."""
    value, shapes, starts, loc, attn = make_operands("cpu", 2, 4, requires_grad=False)
    stacked = torch.stack([shapes, shapes])
    with pytest.raises(RuntimeError, match="spatial_shapes"):
        torch.vmap(lambda s: msda(value, s, starts, loc, attn))(stacked)


@pytest.mark.gpu
@pytest.mark.parametrize(("name", "method"), CASES)
def test_vmap_folds_into_the_batch(device, name, method):
    """vmap over a stack of 3 batches (and over value alone, with locations and
    weights shared) equals the per-batch calls, gradients included."""
    value, shapes, starts, loc, attn = make_operands(device, 2, 5, requires_grad=False)
    values = torch.stack([value, value * 2, value - 1])
    locs = torch.stack([loc, loc.flip(1), loc * 0.5 + 0.2])
    attns = torch.stack([attn, attn.flip(1), attn * 2])

    def call(v, lo, a):
        return msda(v, shapes, starts, lo, a, method=method)

    mapped = torch.vmap(call)(values, locs, attns)
    each = torch.stack([call(v, lo, a) for v, lo, a in zip(values, locs, attns)])
    torch.testing.assert_close(mapped, each, rtol=1e-5, atol=1e-6)
    shared = torch.vmap(call, in_dims=(0, None, None))(values, loc, attn)
    torch.testing.assert_close(shared, torch.stack([call(v, loc, attn) for v in values]), rtol=1e-5, atol=1e-6)
    leaves = [t.clone().requires_grad_(True) for t in (values, locs, attns)]
    torch.vmap(call)(*leaves).square().sum().backward()
    ref_leaves = [t.clone().requires_grad_(True) for t in (values, locs, attns)]
    torch.stack([call(v, lo, a) for v, lo, a in zip(*ref_leaves)]).square().sum().backward()
    for got, want in zip(leaves, ref_leaves):
        torch.testing.assert_close(got.grad, want.grad, rtol=1e-4, atol=1e-5)
