"""msda_backward_no_alloc, the backward that allocates nothing, against
msda_backward_workspace through the C ABI.

The entry point has no counterpart in the reference: it serves callers that cannot
allocate device memory (code under HIP graph capture, serving loops, harnesses that
forbid hipMalloc). Its workspace is a static device array of 64 MiB that every call
on a device shares, so the checks run two calls in a row, the second on a smaller
problem, to show that nothing the first call left there leaks into the second.
The bar is the workspace call's: location and weight gradients bit-equal (the same
kernel on the same inputs), grad_value the same sums in another order (float32 1e-4,
16-bit 2e-2 of the largest element, the parity suite's tolerances), and both within
those tolerances of the float64 C oracle on the smaller problem.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from deformops_amd.backends.hip import _lib
from tests.workloads import make_workload

F32, BF16, F16 = torch.float32, torch.bfloat16, torch.float16
BWD_TOL = {F32: 1e-4, BF16: 2e-2, F16: 2e-2}
SCRATCH_BYTES = 64 << 20


def rel_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    actual = actual.detach().to("cpu", torch.float64).reshape(expected.shape)
    expected = expected.detach().to("cpu", torch.float64)
    scale = expected.abs().max().item()
    diff = (actual - expected).abs().max().item()
    return diff / scale if scale else diff


def call(lib, entry: str, w, grads, flags: int) -> None:
    value, shapes, starts, loc, attn = w.operands(softmax=bool(flags & _lib.FLAG_SOFTMAX))
    B, S, H, D, Q, L, P = w.sizes  # noqa: N806
    args = (value.data_ptr(), _lib.DTYPE_CODES[value.dtype], shapes.data_ptr(), starts.data_ptr(),
            _lib.INDEX_CODES[shapes.dtype], loc.data_ptr(), _lib.DTYPE_CODES[loc.dtype], attn.data_ptr(),
            w.grad_output.data_ptr(), *(t.data_ptr() for t in grads), B, S, H, D, Q, L, P, flags)
    stream = torch.cuda.current_stream().cuda_stream
    if entry == "no_alloc":
        lib.check(lib.backward_no_alloc(*args, stream))
    else:
        size = lib.workspace_size(value.dtype, B, S, H, D, Q, L, P, flags)
        ws = torch.empty(size, dtype=torch.uint8, device=value.device)
        lib.check(lib.backward_workspace(*args, ws.data_ptr(), size, stream))


@pytest.mark.gpu
@pytest.mark.parametrize("softmax", [False, True], ids=["linear", "softmax"])
@pytest.mark.parametrize("dtype", [BF16, F16, F32], ids=["bf16", "f16", "f32"])
def test_no_alloc_backward_matches_the_workspace_backward(device, dtype, softmax):
    lib = _lib.load()
    flags = _lib.FLAG_SOFTMAX if softmax else 0
    # The headline problem (B = 4, Q = 21,504; in float32 its workspace nearly fills
    # the scratch), then a smaller one on top of what it left there.
    works = [make_workload(4).to(device, dtype), make_workload(2, batch=1, queries=3000, seed=7).to(device, dtype)]
    for i, w in enumerate(works):
        # The scratch holds the indices and the counters (the linear method's workspace);
        # the softmax statistics' region of the workspace entry is not needed here.
        assert lib.workspace_size(dtype, *w.sizes, 0) <= SCRATCH_BYTES
        want = [torch.empty_like(t) for t in (w.value, w.sampling_locations, w.attention_weights)]
        got = [torch.full_like(t, float("nan")) for t in want]
        call(lib, "workspace", w, want, flags)
        call(lib, "no_alloc", w, got, flags)
        torch.cuda.synchronize()
        label = f"call {i} {tuple(w.sizes)}"
        assert rel_err(got[0], want[0]) <= BWD_TOL[dtype], label
        torch.testing.assert_close(got[1], want[1], rtol=0, atol=0, msg=label)
        torch.testing.assert_close(got[2], want[2], rtol=0, atol=0, msg=label)
    value, shapes, starts, loc, attn = (t.cpu() for t in works[1].operands(softmax=softmax))
    ref = oracle.backward(value, shapes, starts, loc, attn, works[1].grad_output.cpu(), softmax=softmax)
    for g, r in zip(got, ref):
        assert rel_err(g, r.reshape(g.shape)) <= BWD_TOL[dtype]


@pytest.mark.gpu
def test_no_alloc_backward_accumulates_and_repeats(device):
    """MSDA_ACCUMULATE_GRAD_VALUE adds into the caller's grad_value, and a repeated call
    on the same problem gives the same location and weight gradients."""
    lib = _lib.load()
    w = make_workload(2, batch=1, queries=2500, seed=3).to(device, BF16)
    base = torch.randn_like(w.value)
    want = [torch.empty_like(t) for t in (w.value, w.sampling_locations, w.attention_weights)]
    call(lib, "workspace", w, want, 0)
    for _ in range(2):
        got = [base.clone(), torch.empty_like(want[1]), torch.empty_like(want[2])]
        call(lib, "no_alloc", w, got, _lib.FLAG_ACCUMULATE_GRAD_VALUE)
        torch.cuda.synchronize()
        assert rel_err(got[0], base.double() + want[0].double()) <= BWD_TOL[BF16]
        torch.testing.assert_close(got[1], want[1], rtol=0, atol=0)
        torch.testing.assert_close(got[2], want[2], rtol=0, atol=0)


def test_no_alloc_backward_rejects_sizes_beyond_the_scratch():
    """A problem whose workspace exceeds the 64 MiB scratch fails before any launch
    (host-side check; no GPU needed), naming the bytes it needs."""
    lib = _lib.load()
    # 2^23 + 2^13 samples in float32: 8 bytes each, just over 64 MiB.
    sizes = (1, 1000, 8, 32, 2 ** 20 + 2 ** 10, 1, 1)
    assert lib.workspace_size(F32, *sizes) > SCRATCH_BYTES
    p = 1  # never dereferenced: the call fails first
    rc = lib.backward_no_alloc(*(p, 0, p, p, 0, p, 0, p, p, p, p, p), *sizes, 0, None)
    assert rc == 1  # MSDA_ERR_INVALID
    message = lib.cdll.msda_last_error().decode()
    assert "scratch" in message and str(lib.workspace_size(F32, *sizes)) in message, message
    # At 2^23 samples it fits.
    assert lib.workspace_size(F32, 1, 1000, 8, 32, 2 ** 20, 1, 1) <= SCRATCH_BYTES
