"""TEST INFRASTRUCTURE ONLY: CPU oracles of the MSDA operator.

Only tests/, bench.py's cpu_baseline leg and __graft_entry__.smoke() import this
package, and only as the checker; the product path (deformops_amd) never does.

- :func:`forward` / :func:`backward`: the C restatement (msda_oracle.c), float64.
- :mod:`oracle.eager`: torch restatement of the reference eager backend; its
  autograd is an independent derivation of the backward; also the CPU baseline.
- :mod:`oracle.grid_sample_ref`: the reference's grid_sample definition.
"""

from __future__ import annotations

import ctypes
import threading

import torch
from torch import Tensor

from .build import LIBRARY, build

__all__ = ["backward", "forward", "load"]

_lock = threading.Lock()
_cdll: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the C oracle, compiling it with gcc first if it is not built."""
    global _cdll  # noqa: PLW0603
    with _lock:
        if _cdll is None:
            path = LIBRARY if LIBRARY.exists() else build()
            lib = ctypes.CDLL(str(path))
            P, L = ctypes.c_void_p, ctypes.c_int64
            lib.msda_oracle_forward.argtypes = [P] * 6 + [L] * 7 + [ctypes.c_int, ctypes.c_int]
            lib.msda_oracle_forward.restype = ctypes.c_int
            lib.msda_oracle_backward.argtypes = [P] * 9 + [L] * 7 + [ctypes.c_int, ctypes.c_int]
            lib.msda_oracle_backward.restype = ctypes.c_int
            _cdll = lib
    return _cdll


def _prep(value: Tensor, spatial_shapes: Tensor, level_start_index: Tensor, loc: Tensor, attn: Tensor):
    B, S, H, D = value.shape
    Q, L, P = loc.shape[1], spatial_shapes.shape[0], loc.shape[4]
    f64 = lambda t: t.detach().to("cpu", torch.float64).contiguous()  # noqa: E731
    i64 = lambda t: t.detach().to("cpu", torch.int64).contiguous()  # noqa: E731
    return (
        (int(B), int(S), int(H), int(D), int(Q), int(L), int(P)),
        f64(value),
        i64(spatial_shapes),
        i64(level_start_index),
        f64(loc),
        f64(attn.reshape(B, Q, H, L * P)),
    )


def forward(
    value: Tensor,
    spatial_shapes: Tensor,
    level_start_index: Tensor,
    sampling_locations: Tensor,
    attention_weights: Tensor,
    *,
    softmax: bool = False,
    pixel_f32: bool | None = None,
) -> Tensor:
    """MSDA forward in float64 on the CPU: ``(B, Q, H * D)``.

    ``pixel_f32`` (default: unless value is float64) rounds the pixel map in float32.
    """
    if pixel_f32 is None:
        pixel_f32 = value.dtype != torch.float64
    (B, S, H, D, Q, L, P), v, sh, st, lc, at = _prep(
        value, spatial_shapes, level_start_index, sampling_locations, attention_weights
    )
    out = torch.empty((B, Q, H * D), dtype=torch.float64)
    rc = load().msda_oracle_forward(
        v.data_ptr(), sh.data_ptr(), st.data_ptr(), lc.data_ptr(), at.data_ptr(), out.data_ptr(),
        B, S, H, D, Q, L, P, int(softmax), int(pixel_f32),
    )
    if rc != 0:
        raise MemoryError("msda_oracle_forward failed")
    return out


def backward(
    value: Tensor,
    spatial_shapes: Tensor,
    level_start_index: Tensor,
    sampling_locations: Tensor,
    attention_weights: Tensor,
    grad_output: Tensor,
    *,
    softmax: bool = False,
    pixel_f32: bool | None = None,
) -> tuple[Tensor, Tensor, Tensor]:
    """Float64 gradients ``(grad_value, grad_loc, grad_attn)``; grad_attn is flat ``(B, Q, H, L*P)``."""
    if pixel_f32 is None:
        pixel_f32 = value.dtype != torch.float64
    (B, S, H, D, Q, L, P), v, sh, st, lc, at = _prep(
        value, spatial_shapes, level_start_index, sampling_locations, attention_weights
    )
    go = grad_output.detach().to("cpu", torch.float64).reshape(B, Q, H * D).contiguous()
    gv = torch.empty((B, S, H, D), dtype=torch.float64)
    gl = torch.empty((B, Q, H, L, P, 2), dtype=torch.float64)
    ga = torch.empty((B, Q, H, L * P), dtype=torch.float64)
    rc = load().msda_oracle_backward(
        v.data_ptr(), sh.data_ptr(), st.data_ptr(), lc.data_ptr(), at.data_ptr(), go.data_ptr(),
        gv.data_ptr(), gl.data_ptr(), ga.data_ptr(),
        B, S, H, D, Q, L, P, int(softmax), int(pixel_f32),
    )
    if rc != 0:
        raise MemoryError("msda_oracle_backward failed")
    return gv, gl, ga

