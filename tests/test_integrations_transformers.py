"""The Hugging Face integration: ``run_msda``, module patching, and the drop-in
attention modules against the upstream ``transformers`` implementations
(reference ``integrations/transformers.py``, ``integrations/_ops.py``,
``integrations/_patch.py``; its model tests ``tests/deformops/models/test_mask2former.py``
and ``test_deformable_detr.py``).

Models are small random-weight configurations built offline. On the CPU the
replacements run on the eager oracle (an ``MSDABackend`` adapter), which checks the
host logic; the GPU tests run them on the HIP kernels against upstream's own
``grid_sample`` implementation.
"""

from __future__ import annotations

import copy

import pytest
import torch
from torch import nn

pytest.importorskip("transformers")

from transformers import (  # noqa: E402
    DeformableDetrConfig,
    DeformableDetrForObjectDetection,
    Mask2FormerConfig,
    Mask2FormerForUniversalSegmentation,
    ResNetConfig,
)
from transformers.models.deformable_detr import modeling_deformable_detr as hf_detr  # noqa: E402
from transformers.models.mask2former import modeling_mask2former as hf_m2f  # noqa: E402
from transformers.models.swin.configuration_swin import SwinConfig  # noqa: E402

from deformops_amd.core.errors import NoBackendError  # noqa: E402
from deformops_amd.core.runtime import Method  # noqa: E402
from deformops_amd.integrations import transformers as integ  # noqa: E402
from deformops_amd.integrations._ops import run_msda  # noqa: E402
from deformops_amd.integrations._patch import patch_modules, replace_module_recursively  # noqa: E402
from deformops_amd.registry import Backend, msda  # noqa: E402
from oracle.eager import eager_msda  # noqa: E402

F32 = torch.float32
UpstreamM2F = hf_m2f.Mask2FormerPixelDecoderEncoderMultiscaleDeformableAttention
UpstreamCore = hf_detr.MultiScaleDeformableAttention


class RecordingOracleBackend:
    """An ``MSDABackend`` over the eager oracle that records each call's arguments."""

    name = "eager-oracle"

    def __init__(self) -> None:
        self.calls: list[dict] = []

    def supports(self, context) -> bool:  # noqa: ANN001, ARG002
        return True

    def forward(self, value, spatial_shapes, level_start_index, loc, weights, chunk_step, method):  # noqa: ANN001, ANN201, PLR0913
        self.calls.append({"starts": level_start_index.tolist(), "chunk_step": chunk_step,
                           "method": Method(method), "weights_shape": tuple(weights.shape)})
        return eager_msda(value, spatial_shapes, level_start_index, loc, weights,
                          softmax=Method(method) is Method.SOFTMAX)


def tiny_mask2former() -> nn.Module:
    backbone = SwinConfig(image_size=64, patch_size=4, embed_dim=8, depths=[1, 1, 1, 1],
                          num_heads=[1, 1, 1, 1], window_size=2, out_indices=[1, 2, 3, 4])
    config = Mask2FormerConfig(feature_size=32, mask_feature_size=32, hidden_dim=32,
                               num_attention_heads=4, encoder_layers=2, decoder_layers=1,
                               encoder_feedforward_dim=64, dim_feedforward=64, num_queries=10,
                               backbone_config=backbone)
    return Mask2FormerForUniversalSegmentation(config).eval()


def tiny_deformable_detr() -> nn.Module:
    config = DeformableDetrConfig(
        backbone_config=ResNetConfig(embedding_size=16, hidden_sizes=[16, 24, 32, 48],
                                     depths=[1, 1, 1, 1], out_features=["stage2", "stage3", "stage4"]),
        use_pretrained_backbone=False, use_timm_backbone=False, d_model=32, encoder_layers=1,
        decoder_layers=2, encoder_attention_heads=4, decoder_attention_heads=4,
        encoder_ffn_dim=64, decoder_ffn_dim=64, num_queries=10, num_feature_levels=4)
    return DeformableDetrForObjectDetection(config).eval()


MODELS = {
    # name: (factory, image size, outputs, number of attention modules)
    "mask2former": (tiny_mask2former, 64,
                    lambda o: (o.class_queries_logits, o.masks_queries_logits), 2),
    "deformable_detr": (tiny_deformable_detr, 128, lambda o: (o.logits, o.pred_boxes), 3),
}


def generic_sampling(model: nn.Module) -> nn.Module:
    """Random offset and weight projections in every attention module.

    At upstream's initialization the offsets are whole pixels from pixel-centred
    reference points, so every sample sits exactly on a cell boundary, where the
    location gradient jumps and a one-ulp difference in the pixel map picks
    another cell. Random projections put the samples at generic places.
    """
    g = torch.Generator().manual_seed(3)
    for module in model.modules():
        if isinstance(module, (UpstreamM2F, hf_detr.DeformableDetrMultiscaleDeformableAttention)):
            for lin in (module.sampling_offsets, module.attention_weights):
                with torch.no_grad():
                    lin.weight.copy_(torch.randn(lin.weight.shape, generator=g) * 0.1)
                    lin.bias.copy_(torch.randn(lin.bias.shape, generator=g) * 0.5)
    return model


def m2f_inputs(device, *, boxes=False, mask=False, batch=2, embed=32, levels=3, seed=0):
    g = torch.Generator().manual_seed(seed)
    shapes = [(8, 9), (4, 5), (2, 3)][:levels]
    S = sum(h * w for h, w in shapes)
    hidden = torch.randn(batch, S, embed, generator=g)
    coords = 4 if boxes else 2
    ref = torch.rand(batch, S, levels, coords, generator=g) * 0.8 + 0.1
    if boxes:
        ref[..., 2:] *= 0.4
    kwargs = {
        "encoder_hidden_states": hidden,
        "position_embeddings": torch.randn(batch, S, embed, generator=g),
        "reference_points": ref,
        "spatial_shapes_list": shapes,
        "level_start_index": torch.tensor([0, 72, 92][:levels]),
    }
    if mask:
        kwargs["attention_mask"] = torch.rand(batch, S, generator=g) < 0.2
    out = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in kwargs.items()}
    return hidden.to(device), out


def upstream_m2f(seed=0, embed=32, heads=4, levels=3, points=4) -> nn.Module:
    torch.manual_seed(seed)
    module = UpstreamM2F(embed_dim=embed, num_heads=heads, n_levels=levels, n_points=points)
    # Upstream's init zeroes the weight projections; random ones exercise the sampling.
    for lin in (module.sampling_offsets, module.attention_weights):
        nn.init.normal_(lin.weight, std=0.2)
        nn.init.normal_(lin.bias, std=0.5)
    return module


# patch_modules


class Leaf(nn.Module):
    pass


class Inner(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.leaf = Leaf()


class Replacement(nn.Module):
    def __init__(self, old: nn.Module) -> None:
        super().__init__()
        self.kept = old


def test_patch_modules_replaces_nested_and_walks_replacements():
    root = nn.Sequential(Inner(), nn.Sequential(Leaf(), nn.Linear(2, 2)))
    patch_modules(root, [(Inner, Replacement), (Leaf, lambda _old: nn.Identity())])
    assert isinstance(root[0], Replacement)
    # The replacement's children are walked: the Leaf kept inside Inner is swapped too.
    assert isinstance(root[0].kept.leaf, nn.Identity)
    assert isinstance(root[1][0], nn.Identity)
    assert isinstance(root[1][1], nn.Linear)


def test_patch_modules_keeps_a_shared_module_shared():
    shared = Leaf()
    root = nn.Sequential(nn.Sequential(shared), nn.Sequential(shared), shared)
    made = []

    def factory(old):
        made.append(Replacement(old))
        return made[-1]

    patch_modules(root, [(Leaf, factory)])
    assert len(made) == 1
    assert root[0][0] is root[1][0] is root[2] is made[0]
    assert made[0].kept is shared


def test_patch_modules_first_matching_class_wins():
    root = nn.Sequential(Leaf())
    patch_modules(root, [(nn.Module, lambda _old: nn.Identity()), (Leaf, Replacement)])
    assert isinstance(root[0], nn.Identity)


def test_patch_modules_never_replaces_the_root():
    root = Leaf()
    with pytest.raises(RuntimeError, match="strict=False"):
        patch_modules(root, [(Leaf, Replacement)])
    assert patch_modules(root, [(Leaf, Replacement)], strict=False) is root


def test_replace_module_recursively_is_one_class():
    root = nn.Sequential(Leaf(), Leaf())
    assert replace_module_recursively(root, Leaf, lambda _old: nn.Identity()) is root
    assert all(isinstance(m, nn.Identity) for m in root)


# run_msda


def small_operands(levels=((3, 4), (2, 2)), B=2, Q=5, H=2, D=4, P=2, seed=0):
    g = torch.Generator().manual_seed(seed)
    shapes = torch.tensor(levels)
    S = int((shapes[:, 0] * shapes[:, 1]).sum())
    value = torch.randn(B, S, H, D, generator=g)
    loc = torch.rand(B, Q, H, len(levels), P, 2, generator=g)
    attn = torch.rand(B, Q, H, len(levels) * P, generator=g)
    return value, shapes, loc, attn


def test_run_msda_derives_level_starts_and_passes_chunk_step():
    value, shapes, loc, attn = small_operands(levels=((3, 4), (2, 2), (1, 3)))
    backend = RecordingOracleBackend()
    out = run_msda(value, shapes, None, loc, attn, chunk_step=7, backend=backend)
    assert backend.calls == [{"starts": [0, 12, 16], "chunk_step": 7, "method": Method.LINEAR,
                              "weights_shape": tuple(attn.shape)}]
    starts = torch.tensor([0, 12, 16])
    torch.testing.assert_close(out, eager_msda(value, shapes, starts, loc, attn), rtol=0, atol=0)
    run_msda(value, shapes, starts, loc, attn, chunk_step=3, backend=backend, method=Method.SOFTMAX)
    assert backend.calls[-1]["method"] is Method.SOFTMAX


def test_run_msda_cpu_tensors_reach_the_registry():
    """CPU tensors run the eager backend by default; HIP declines them."""
    value, shapes, loc, attn = small_operands()
    starts = torch.cat([shapes.new_zeros(1), (shapes[:, 0] * shapes[:, 1]).cumsum(0)[:-1]])
    out = run_msda(value, shapes, None, loc, attn, chunk_step=64, backend=None)
    torch.testing.assert_close(out, eager_msda(value, shapes, starts, loc, attn), rtol=1e-5, atol=1e-6)
    with pytest.raises((NoBackendError, RuntimeError)):
        run_msda(value, shapes, None, loc, attn, chunk_step=64, backend=Backend.HIP)


# the drop-in modules on the CPU (oracle backend)


def test_mask2former_replacement_shares_the_projections():
    old = upstream_m2f()
    new = integ.Mask2FormerPixelDecoderEncoderMultiscaleDeformableAttention(old)
    for name in ("sampling_offsets", "attention_weights", "value_proj", "output_proj"):
        assert getattr(new, name) is getattr(old, name)
    assert new.chunk_step == old.im2col_step
    assert (new.n_heads, new.n_levels, new.n_points, new.d_model) == (4, 3, 4, 32)
    assert isinstance(new, UpstreamM2F)


@pytest.mark.parametrize(("boxes", "mask"), [(False, False), (True, False), (False, True)])
def test_mask2former_attention_matches_upstream_on_cpu(boxes, mask):
    old = upstream_m2f()
    backend = RecordingOracleBackend()
    new = integ.Mask2FormerPixelDecoderEncoderMultiscaleDeformableAttention(old, backend=backend)
    hidden, kwargs = m2f_inputs("cpu", boxes=boxes, mask=mask)
    with torch.no_grad():
        out_up, w_up = old(hidden, **kwargs)
        out_new, w_new = new(hidden, **kwargs)
    torch.testing.assert_close(out_new, out_up, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(w_new, w_up, rtol=0, atol=0)
    assert backend.calls[0]["chunk_step"] == 128
    assert backend.calls[0]["method"] is Method.LINEAR


def test_mask2former_attention_takes_a_spatial_shapes_tensor():
    old = upstream_m2f()
    new = integ.Mask2FormerPixelDecoderEncoderMultiscaleDeformableAttention(old, backend=RecordingOracleBackend())
    hidden, kwargs = m2f_inputs("cpu")
    listed = new(hidden, **kwargs)[0]
    kwargs["spatial_shapes"] = torch.tensor(kwargs.pop("spatial_shapes_list"))
    torch.testing.assert_close(new(hidden, **kwargs)[0], listed, rtol=0, atol=0)


@pytest.mark.parametrize(
    ("change", "fragment"),
    [
        ({"spatial_shapes_list": None}, "spatial_shapes"),
        ({"reference_points": None}, "reference_points are required"),
        ({"encoder_hidden_states": None}, "encoder_hidden_states"),
        ({"spatial_shapes_list": [(8, 9), (4, 5), (2, 2)]}, "align the spatial shapes"),
        ({"reference_points": torch.rand(2, 98, 3, 3)}, "must be 2 or 4"),
    ],
)
def test_mask2former_attention_errors(change, fragment):
    new = integ.Mask2FormerPixelDecoderEncoderMultiscaleDeformableAttention(
        upstream_m2f(), backend=RecordingOracleBackend())
    hidden, kwargs = m2f_inputs("cpu")
    kwargs.update(change)
    with pytest.raises(ValueError, match=fragment):
        new(hidden, **kwargs)


def test_core_replacement_matches_upstream_on_cpu():
    backend = RecordingOracleBackend()
    new = integ.MultiScaleDeformableAttention(backend=backend)
    value, shapes, loc, attn = small_operands(levels=((5, 6), (3, 3)), P=3)
    B, Q, H, L, P, _ = loc.shape
    weights = torch.softmax(attn, -1).view(B, Q, H, L, P)
    starts = torch.tensor([0, 30])
    args = (value, shapes, [tuple(s) for s in shapes.tolist()], starts, loc, weights, 64)
    torch.testing.assert_close(new(*args), UpstreamCore()(*args), rtol=1e-5, atol=1e-6)
    assert backend.calls[0]["chunk_step"] == 64
    assert backend.calls[0]["weights_shape"] == (B, Q, H, L, P)


def test_strict_patch_of_a_model_without_attention_raises():
    with pytest.raises(RuntimeError, match="MultiScaleDeformableAttention"):
        integ.patch(nn.Sequential(nn.Linear(2, 2)))
    model = nn.Sequential(nn.Linear(2, 2))
    assert integ.patch(model, strict=False) is model


@pytest.mark.parametrize("name", sorted(MODELS))
def test_patched_model_matches_upstream_on_cpu(name):
    factory, size, outputs_of, count = MODELS[name]
    torch.manual_seed(0)
    upstream = generic_sampling(factory())
    backend = RecordingOracleBackend()
    patched = integ.patch(copy.deepcopy(upstream), backend=backend)
    kinds = (integ.MultiScaleDeformableAttention,
             integ.Mask2FormerPixelDecoderEncoderMultiscaleDeformableAttention)
    assert sum(isinstance(m, kinds) for m in patched.modules()) == count
    image = torch.randn(1, 3, size, size, generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        expected = outputs_of(upstream(image))
        actual = outputs_of(patched(image))
    assert len(backend.calls) == count
    for a, e in zip(actual, expected):
        torch.testing.assert_close(a, e, rtol=1e-4, atol=1e-4)


# on the GPU: the HIP kernels against upstream's grid_sample implementation


def grads_of(module: nn.Module, tensors) -> list[torch.Tensor]:
    return [p.grad.clone() for p in module.parameters() if p.grad is not None] + \
        [t.grad.clone() for t in tensors]


@pytest.mark.gpu
@pytest.mark.parametrize(("boxes", "mask"), [(False, False), (True, False), (False, True)])
def test_mask2former_attention_matches_upstream_on_gpu(device, boxes, mask):
    old = upstream_m2f().to(device)
    twin = copy.deepcopy(old)
    new = integ.Mask2FormerPixelDecoderEncoderMultiscaleDeformableAttention(twin)
    runs = []
    for module in (old, new):
        hidden, kwargs = m2f_inputs(device, boxes=boxes, mask=mask)
        hidden.requires_grad_(True)
        kwargs["encoder_hidden_states"].requires_grad_(True)
        kwargs["reference_points"].requires_grad_(True)
        out, weights = module(hidden, **kwargs)
        out.backward(torch.randn(out.shape, generator=torch.Generator().manual_seed(5)).to(device))
        runs.append((out.detach(), weights.detach(), grads_of(
            module, [hidden, kwargs["encoder_hidden_states"], kwargs["reference_points"]])))
    (out_up, w_up, g_up), (out_new, w_new, g_new) = runs
    # fp32 tolerances: forward 1e-5, backward 1e-4.
    torch.testing.assert_close(out_new, out_up, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(w_new, w_up, rtol=1e-6, atol=1e-7)
    assert len(g_new) == len(g_up) == 11
    for a, e in zip(g_new, g_up):
        torch.testing.assert_close(a, e, rtol=1e-4, atol=1e-4)


class RecordingRegistryBackend:
    """An ``MSDABackend`` that runs the registry's choice (the HIP kernels) and
    keeps each call's operands and result."""

    name = "recording-registry"

    def __init__(self) -> None:
        self.calls: list[tuple] = []

    def supports(self, context) -> bool:  # noqa: ANN001, ARG002
        return True

    def forward(self, value, spatial_shapes, level_start_index, loc, weights, chunk_step, method):  # noqa: ANN001, ANN201, ARG002, PLR0913
        out = msda(value, spatial_shapes, level_start_index, loc, weights, method=method)
        self.calls.append((value, spatial_shapes, level_start_index, loc, weights, out))
        return out


@pytest.mark.gpu
def test_mask2former_attention_bf16_on_gpu(device):
    """A bf16 module hands bf16 operands to the kernels; their result is checked
    against the oracle on those same operands (bf16 tolerance 2e-2)."""
    backend = RecordingRegistryBackend()
    new = integ.Mask2FormerPixelDecoderEncoderMultiscaleDeformableAttention(
        upstream_m2f().to(device, torch.bfloat16), backend=backend)
    hidden, kwargs = m2f_inputs(device)
    half = {k: (v.to(torch.bfloat16) if isinstance(v, torch.Tensor) and v.is_floating_point() else v)
            for k, v in kwargs.items()}
    with torch.no_grad():
        out, weights = new(hidden.to(torch.bfloat16), **half)
    assert out.dtype == weights.dtype == torch.bfloat16
    (value, shapes, starts, loc, attn, result), = backend.calls
    assert value.dtype == attn.dtype == loc.dtype == torch.bfloat16
    expected = eager_msda(*(t.cpu().double() if t.is_floating_point() else t.cpu()
                            for t in (value, shapes, starts, loc, attn)))
    err = (result.cpu().double() - expected).abs().max() / expected.abs().max()
    assert err < 2e-2


@pytest.mark.gpu
def test_core_replacement_matches_upstream_on_gpu(device):
    value, shapes, loc, attn = small_operands(levels=((17, 23), (9, 12), (5, 6), (3, 3)), B=2, Q=300,
                                              H=4, D=8, P=4)
    B, Q, H, L, P, _ = loc.shape
    starts = torch.cat([torch.zeros(1, dtype=torch.long), (shapes[:, 0] * shapes[:, 1]).cumsum(0)[:-1]])
    runs = []
    for module in (UpstreamCore(), integ.MultiScaleDeformableAttention()):
        v = value.to(device).requires_grad_(True)
        lo = (loc * 1.2 - 0.1).to(device).requires_grad_(True)
        w = torch.softmax(attn, -1).view(B, Q, H, L, P).to(device).requires_grad_(True)
        out = module(v, shapes.to(device), [tuple(s) for s in shapes.tolist()], starts.to(device), lo, w, 64)
        out.backward(torch.ones_like(out))
        runs.append((out.detach(), v.grad, lo.grad, w.grad))
    for a, e in zip(runs[1], runs[0]):
        torch.testing.assert_close(a, e, rtol=1e-4, atol=1e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(MODELS))
def test_patched_model_matches_upstream_on_gpu(device, name):
    factory, size, outputs_of, count = MODELS[name]
    torch.manual_seed(0)
    upstream = generic_sampling(factory()).to(device)
    patched = integ.patch(copy.deepcopy(upstream))
    image = torch.randn(1, 3, size, size, generator=torch.Generator().manual_seed(1)).to(device)
    expected = outputs_of(upstream(image))
    actual = outputs_of(patched(image))
    for a, e in zip(actual, expected):
        torch.testing.assert_close(a, e, rtol=1e-4, atol=1e-4)
    sum(o.float().sum() for o in expected).backward()
    sum(o.float().sum() for o in actual).backward()
    compared = 0
    for (name_up, p_up), (name_new, p_new) in zip(upstream.named_parameters(), patched.named_parameters()):
        assert name_up == name_new
        if p_up.grad is None:
            assert p_new.grad is None
            continue
        torch.testing.assert_close(p_new.grad, p_up.grad, rtol=1e-3, atol=1e-4,
                                   msg=lambda m, n=name_up: f"{n}: {m}")
        compared += 1
    assert compared > 0
