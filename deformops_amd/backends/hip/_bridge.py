r"""Private operators of the HIP backend, with their autograd and fake kernels.

Mirrors the reference CUDA bridge (sources/deformops/backends/cuda/_msda_bridge.py:
146-492 and _schema.py:18-29): four operators in their own namespace with the
reference's argument lists,

    deformops_hip::msda[_softmax]_forward(value, spatial_shapes, level_start_index,
        loc, attn, chunk_step, K, channels_per_thread, threads_per_block) -> out
    deformops_hip::msda[_softmax]_backward(..., grad_output, chunk_step, K,
        channels_per_thread, threads_per_block) -> (grad_value, grad_loc, grad_attn)

each implemented for GPU tensors by one call into libdeformops_amd.so. Unlike the
reference's float32-accumulator configuration, the backward hands the kernel the
16-bit tensors as they are: there is no float32 upcast, no float32 scratch
``grad_value`` and no copy back; each element of ``grad_value`` is summed in fp32
by its one owner and stored once. ``chunk_step``, ``channels_per_thread`` and
``threads_per_block`` are accepted and ignored (the kernels pick their own layout);
``K`` must equal the points axis of ``loc``.
"""

from __future__ import annotations

import contextlib
import functools
from typing import Any

import torch
import torch.library
from torch import Tensor

from ...core.runtime import Method
from ...registry import MSDAContext, resolve_msda_attn
from . import _lib

__all__ = [
    "NAMESPACE",
    "Backend",
    "backward_op",
    "forward",
    "forward_op",
    "supports_context",
]

NAMESPACE = "deformops_hip"

_FORWARD_SCHEMA = (
    "(Tensor value, Tensor spatial_shapes, Tensor level_start_index, Tensor loc, "
    "Tensor attn, int chunk_step, int K, int channels_per_thread, "
    "int threads_per_block) -> Tensor"
)
_BACKWARD_SCHEMA = (
    "(Tensor value, Tensor spatial_shapes, Tensor level_start_index, Tensor loc, "
    "Tensor attn, Tensor grad_output, int chunk_step, int K, int channels_per_thread, "
    "int threads_per_block) -> (Tensor, Tensor, Tensor)"
)

_SUPPORTED_DTYPES = (torch.float32, torch.float16, torch.bfloat16, torch.float64)

#: Held for the life of the process: a collected Library unregisters its operators.
_LIBRARY = torch.library.Library(NAMESPACE, "DEF")


# Operand normalization.


def _index_tables(spatial_shapes: Tensor, level_start_index: Tensor) -> tuple[Tensor, Tensor]:
    """Both tables as one of the kernel's index dtypes (int32 kept, others int64)."""
    if spatial_shapes.dtype == level_start_index.dtype and spatial_shapes.dtype in _lib.INDEX_CODES:
        return spatial_shapes.contiguous(), level_start_index.contiguous()
    return (
        spatial_shapes.to(torch.int64).contiguous(),
        level_start_index.to(torch.int64).contiguous(),
    )


def _location_dtype(value_dtype: torch.dtype, loc_dtype: torch.dtype) -> torch.dtype:
    """Locations run as float32 or the value dtype; float64 values take float64."""
    if value_dtype == torch.float64:
        return torch.float64
    if loc_dtype in (torch.float32, value_dtype):
        return loc_dtype
    return torch.float32


def _sizes(value: Tensor, spatial_shapes: Tensor, loc: Tensor) -> tuple[int, ...]:
    B, S, H, D = value.shape
    Q, L, P = loc.shape[1], spatial_shapes.shape[0], loc.shape[4]
    return int(B), int(S), int(H), int(D), int(Q), int(L), int(P)


def _check_points(loc: Tensor, K: int) -> None:  # noqa: N803
    if K != loc.shape[4]:
        msg = f"K={K} does not match the {loc.shape[4]} points per level of loc"
        raise ValueError(msg)


def _on_device(device: torch.device) -> Any:
    """The device's context when it is not the current one (the library launches on
    the current device)."""
    return contextlib.nullcontext() if device.index == torch.cuda.current_device() else torch.cuda.device(device)


# Device kernels. The launch functions take operands as _forward_impl and
# _backward_impl normalize them (contiguous, level tables in a kernel index dtype,
# locations in a kernel location dtype, weights in the value dtype).


def _launch_forward(value: Tensor, shapes: Tensor, starts: Tensor, loc: Tensor, attn: Tensor, *,
                    softmax: bool) -> Tensor:
    B, S, H, D, Q, L, P = _sizes(value, shapes, loc)
    out = torch.empty((B, Q, H * D), dtype=value.dtype, device=value.device)
    lib = _lib.load()
    with _on_device(value.device):
        status = lib.forward(
            value.data_ptr(), _lib.DTYPE_CODES[value.dtype],
            shapes.data_ptr(), starts.data_ptr(), _lib.INDEX_CODES[shapes.dtype],
            loc.data_ptr(), _lib.DTYPE_CODES[loc.dtype],
            attn.data_ptr(), out.data_ptr(),
            B, S, H, D, Q, L, P,
            _lib.FLAG_SOFTMAX if softmax else 0,
            torch._C._cuda_getCurrentRawStream(value.device.index),  # noqa: SLF001
        )
    lib.check(status)
    return out


def _launch_backward(value: Tensor, shapes: Tensor, starts: Tensor, loc: Tensor, attn: Tensor,
                     grad_output: Tensor, *, softmax: bool) -> tuple[Tensor, Tensor, Tensor]:
    B, S, H, D, Q, L, P = _sizes(value, shapes, loc)
    grad_c = grad_output.to(value.dtype).contiguous()
    grad_value = torch.empty_like(value)
    grad_loc = torch.empty_like(loc)
    grad_attn = torch.empty_like(attn)
    lib = _lib.load()
    # The sort's scratch in a workspace of its own (the caching allocator's blocks are
    # 512-byte aligned), so that the location and weight gradients need not wait for it.
    workspace = torch.empty(_workspace_bytes(value.dtype, B, S, H, Q, L, P, softmax), dtype=torch.uint8,
                            device=value.device)
    with _on_device(value.device):
        status = lib.backward_workspace(
            value.data_ptr(), _lib.DTYPE_CODES[value.dtype],
            shapes.data_ptr(), starts.data_ptr(), _lib.INDEX_CODES[shapes.dtype],
            loc.data_ptr(), _lib.DTYPE_CODES[loc.dtype],
            attn.data_ptr(), grad_c.data_ptr(),
            grad_value.data_ptr(), grad_loc.data_ptr(), grad_attn.data_ptr(),
            B, S, H, D, Q, L, P,
            _lib.FLAG_SOFTMAX if softmax else 0,
            workspace.data_ptr(), workspace.numel(),
            torch._C._cuda_getCurrentRawStream(value.device.index),  # noqa: SLF001
        )
    lib.check(status)
    return grad_value, grad_loc, grad_attn


@functools.lru_cache(maxsize=256)
def _workspace_bytes(dtype: torch.dtype, B: int, S: int, H: int, Q: int, L: int, P: int,  # noqa: N803
                     softmax: bool) -> int:
    """msda_backward_workspace_size for these sizes, asked of the library once per shape."""
    return _lib.load().workspace_size(dtype, B, S, H, 0, Q, L, P, _lib.FLAG_SOFTMAX if softmax else 0)


def _normalized(value: Tensor, spatial_shapes: Tensor, level_start_index: Tensor, loc: Tensor,
                attn: Tensor) -> tuple[Tensor, ...]:
    shapes, starts = _index_tables(spatial_shapes, level_start_index)
    return (value.contiguous(), shapes, starts, loc.to(_location_dtype(value.dtype, loc.dtype)).contiguous(),
            attn.to(value.dtype).contiguous())


def _forward_impl(
    value: Tensor, spatial_shapes: Tensor, level_start_index: Tensor, loc: Tensor,
    attn: Tensor, K: int, *, softmax: bool,  # noqa: N803
) -> Tensor:
    _check_points(loc, K)
    return _launch_forward(*_normalized(value, spatial_shapes, level_start_index, loc, attn), softmax=softmax)


def _backward_impl(
    value: Tensor, spatial_shapes: Tensor, level_start_index: Tensor, loc: Tensor,
    attn: Tensor, grad_output: Tensor, K: int, *, softmax: bool,  # noqa: N803
) -> tuple[Tensor, Tensor, Tensor]:
    _check_points(loc, K)
    operands = _normalized(value, spatial_shapes, level_start_index, loc, attn)
    grad_value, grad_loc, grad_attn = _launch_backward(*operands, grad_output, softmax=softmax)
    return grad_value, grad_loc.to(loc.dtype), grad_attn.to(attn.dtype)


# Operator registration.


def _define(prefix: str, *, softmax: bool) -> tuple[Any, Any]:
    fwd_name, bwd_name = f"{prefix}_forward", f"{prefix}_backward"
    _LIBRARY.define(f"{fwd_name}{_FORWARD_SCHEMA}")
    _LIBRARY.define(f"{bwd_name}{_BACKWARD_SCHEMA}")

    def forward_kernel(value, spatial_shapes, level_start_index, loc, attn,  # noqa: ANN001, ANN202, PLR0913
                       chunk_step, K, channels_per_thread, threads_per_block):  # noqa: ARG001, N803
        return _forward_impl(value, spatial_shapes, level_start_index, loc, attn, K, softmax=softmax)

    def backward_kernel(value, spatial_shapes, level_start_index, loc, attn, grad_output,  # noqa: ANN001, ANN202, PLR0913
                        chunk_step, K, channels_per_thread, threads_per_block):  # noqa: ARG001, N803
        return _backward_impl(
            value, spatial_shapes, level_start_index, loc, attn, grad_output, K, softmax=softmax
        )

    _LIBRARY.impl(fwd_name, forward_kernel, "CUDA")
    _LIBRARY.impl(bwd_name, backward_kernel, "CUDA")

    def forward_fake(value, spatial_shapes, level_start_index, loc, attn,  # noqa: ANN001, ANN202, PLR0913
                     chunk_step, K, channels_per_thread, threads_per_block):  # noqa: ARG001, N803
        B, _, H, D = value.shape
        return value.new_empty((B, loc.shape[1], H * D))

    def backward_fake(value, spatial_shapes, level_start_index, loc, attn, grad_output,  # noqa: ANN001, ANN202, PLR0913
                      chunk_step, K, channels_per_thread, threads_per_block):  # noqa: ARG001, N803
        return value.new_empty(value.shape), loc.new_empty(loc.shape), attn.new_empty(attn.shape)

    torch.library.register_fake(f"{NAMESPACE}::{fwd_name}", forward_fake, lib=_LIBRARY)
    torch.library.register_fake(f"{NAMESPACE}::{bwd_name}", backward_fake, lib=_LIBRARY)

    fwd_op = getattr(torch.ops.deformops_hip, fwd_name).default
    bwd_op = getattr(torch.ops.deformops_hip, bwd_name).default

    def setup_context(ctx, inputs, output):  # noqa: ANN001, ANN202, ARG001
        value, spatial_shapes, level_start_index, loc, attn, *options = inputs
        ctx.save_for_backward(value, spatial_shapes, level_start_index, loc, attn)
        ctx.options = tuple(options)

    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_output):  # noqa: ANN001, ANN202
        value, spatial_shapes, level_start_index, loc, attn = ctx.saved_tensors
        grad_value, grad_loc, grad_attn = bwd_op(
            value, spatial_shapes, level_start_index, loc, attn, grad_output, *ctx.options
        )
        return grad_value, None, None, grad_loc, grad_attn, None, None, None, None

    torch.library.register_autograd(
        f"{NAMESPACE}::{fwd_name}", backward, setup_context=setup_context, lib=_LIBRARY
    )
    return fwd_op, bwd_op


forward_op, backward_op = _define("msda", softmax=False)
forward_softmax_op, backward_softmax_op = _define("msda_softmax", softmax=True)


class _EagerMSDA(torch.autograd.Function):
    """The private operators' forward and backward for plain eager calls.

    The same two library calls as the registered operators, without the custom-op
    dispatch around each (argument defaults, redispatch, the autograd wrapper), which
    costs more host time than a small call's kernels. Traced, compiled, exported and
    fake calls use the registered operators.
    """

    @staticmethod
    def forward(ctx, value, spatial_shapes, level_start_index, loc, attn, softmax):  # noqa: ANN001, ANN205, PLR0913
        # The operands come normalized from `forward` below.
        ctx.save_for_backward(value, spatial_shapes, level_start_index, loc, attn)
        ctx.softmax = softmax
        return _launch_forward(value, spatial_shapes, level_start_index, loc, attn, softmax=softmax)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_output):  # noqa: ANN001, ANN205
        # The kernels' gradients carry no graph: a second derivative raises, as the
        # reference's CUDA bridge does (cuda/_msda_bridge.py:232).
        value, spatial_shapes, level_start_index, loc, attn = ctx.saved_tensors
        grad_value, grad_loc, grad_attn = _launch_backward(
            value, spatial_shapes, level_start_index, loc, attn, grad_output, softmax=ctx.softmax
        )
        return grad_value, None, None, grad_loc, grad_attn, None


def _plain_eager(*tensors: Tensor) -> bool:
    """Real tensors, no compile / trace, no dispatch or function mode, no functorch wrapper."""
    if torch.compiler.is_compiling() or torch._C._len_torch_dispatch_stack():  # noqa: SLF001
        return False
    if torch._C._is_torch_function_mode_enabled():  # noqa: SLF001
        return False
    wrapped = torch._C._functorch.is_functorch_wrapped_tensor  # noqa: SLF001
    return all(type(t) in (Tensor, torch.nn.Parameter) and not wrapped(t) for t in tensors)


# The adapter surface.


def forward(
    value: Tensor,
    spatial_shapes: Tensor,
    level_start_index: Tensor,
    sampling_locations: Tensor,
    attention_weights: Tensor,
    chunk_step: int = 128,
    *,
    num_points: int | None = None,
    channels_per_thread: int = 0,
    threads_per_block: int = 0,
    softmax: bool = False,
) -> Tensor:
    """Run MSDA on the HIP kernels, differentiably; ``(B, Q, H * D)`` in value's dtype.

    Operands may have any layout and the level tables any integer dtype. Locations
    are kept in float32 or the value dtype (other dtypes are widened to float32,
    and to float64 for float64 values), the autograd of that cast carrying the
    gradient back.
    """
    if value.device.type != "cuda" or torch.version.hip is None:
        msg = (
            f"the HIP MSDA backend runs on ROCm GPU tensors only; got a tensor on "
            f"{value.device}"
        )
        raise RuntimeError(msg)
    if num_points is None:
        num_points = int(sampling_locations.shape[4])
    operands = _normalized(value, spatial_shapes, level_start_index, sampling_locations, attention_weights)
    # The kernels take the operands in their own dtypes: no autocast inside.
    with torch.autocast("cuda", enabled=False) if torch.is_autocast_enabled("cuda") else contextlib.nullcontext():
        if _plain_eager(*operands):
            _check_points(operands[3], num_points)
            return _EagerMSDA.apply(*operands, softmax)
        op = forward_softmax_op if softmax else forward_op
        return op(*operands, chunk_step, num_points, channels_per_thread, threads_per_block)


def _channels_per_lane(dtype: torch.dtype, head_dim: int) -> int:
    cv = 16 // dtype.itemsize
    while cv > 1 and head_dim % cv:
        cv //= 2
    return cv


def supports_context(context: MSDAContext) -> bool:
    """Whether the HIP kernels take a call with this context.

    A ROCm GPU tensor of float32/float16/bfloat16/float64, an image of fewer than
    2^31 elements (S * H * D, when S is known), at most 64 lanes per
    head (``D / channels_per_lane``; D <= 512 for 16-bit values) and one unit's
    staged samples, locations and weights within the 64 KiB LDS budget of a wave
    (the library gives a unit more lanes, and a wave fewer units, until a wave
    fits). Mirrors the library's own launch checks, so dispatch reports
    NoBackendError instead of a launch error; the location width is taken at its
    largest (4 bytes, 8 for float64).
    """
    if context.device.type != "cuda" or torch.version.hip is None:
        return False
    if context.dtype not in _SUPPORTED_DTYPES:
        return False
    samples = context.num_levels * context.num_points
    if samples > 4096:  # noqa: PLR2004
        return False
    head_dim = context.head_dim
    if head_dim == 0:
        return True
    # The kernels index an image's rows with 32-bit offsets: at most 2^31 - 1 elements
    # (S H D) per image, the reference's limit (cuda/include/msda_launch.cuh:85-89).
    if context.num_positions * context.num_heads * head_dim >= 2**31:
        return False
    lanes = head_dim // _channels_per_lane(context.dtype, head_dim)
    if lanes > 64:  # noqa: PLR2004
        return False
    f64 = context.dtype == torch.float64
    staged = 48 if f64 else 32
    value_bytes = context.dtype.itemsize
    loc_bytes = 8 if f64 else 4

    def align16(n: int) -> int:
        return (n + 15) // 16 * 16

    one_unit = align16(16 * context.num_levels + samples * staged) + align16(samples * 2 * loc_bytes)
    return one_unit + align16(samples * value_bytes) <= 64 * 1024


class Backend:
    """Dispatch adapter of the HIP kernels (the MSDABackend protocol)."""

    @property
    def name(self) -> str:
        return "hip"

    def supports(self, context: MSDAContext) -> bool:
        return supports_context(context)

    def forward(
        self,
        value: Tensor,
        spatial_shapes: Tensor,
        level_start_index: Tensor,
        sampling_locations: Tensor,
        attention_weights: Tensor,
        chunk_step: int,
        method: Method,
    ) -> Tensor:
        weights, aggregate = resolve_msda_attn(attention_weights, method)
        return forward(
            value,
            spatial_shapes,
            level_start_index,
            sampling_locations,
            weights,
            chunk_step,
            softmax=aggregate == 1,
        )
