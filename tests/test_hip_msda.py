"""Parity of the HIP MSDA kernels with the CPU oracle, through the drop-in surface.

Each test draws seeded inputs, runs ``deformops_amd.registry.msda`` (forward and
autograd backward) on the GPU, and compares with the float64 C oracle on the same
(rounded) inputs, norm-wise: ``max|actual - expected| / max|expected|`` (the form
of the reference's tests/deformops/test_msda_shared_reduction_gpu.py:75-77).
Tolerances: float32 forward 1e-5, float32 backward 1e-4
(the summation order of grad_value varies), bfloat16 / float16 2e-2 of the float64 result on
the rounded inputs; float64 1e-10.
"""

from __future__ import annotations

import dataclasses
import math

import pytest
import torch

import oracle
from deformops_amd.core.errors import NoBackendError
from deformops_amd.registry import Backend, msda
from oracle.eager import eager_msda
from oracle.grid_sample_ref import grid_sample_msda
from tests.workloads import CONFIGS, make_workload

pytestmark = pytest.mark.gpu

F32, BF16, F16, F64 = torch.float32, torch.bfloat16, torch.float16, torch.float64

FWD_TOL = {F32: 1e-5, F64: 1e-10, BF16: 2e-2, F16: 2e-2}
BWD_TOL = {F32: 1e-4, F64: 1e-10, BF16: 2e-2, F16: 2e-2}


def rel_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    actual = actual.detach().to("cpu", torch.float64).reshape(expected.shape)
    scale = expected.abs().max().item()
    diff = (actual - expected).abs().max().item()
    if scale == 0.0:
        return diff
    return diff / scale


def run_hip(value, shapes, starts, loc, attn, grad_output, *, softmax, backend=None):
    leaves = [t.detach().clone().requires_grad_(True) for t in (value, loc, attn)]
    out = msda(
        leaves[0], shapes, starts, leaves[1], leaves[2],
        method="softmax" if softmax else "linear", backend=backend,
    )
    out.backward(grad_output)
    torch.cuda.synchronize()
    return out.detach(), leaves[0].grad, leaves[1].grad, leaves[2].grad


def check_against_oracle(value, shapes, starts, loc, attn, grad_output, *, softmax, dtype, label=""):
    out, gv, gl, ga = run_hip(value, shapes, starts, loc, attn, grad_output, softmax=softmax)
    assert out.dtype == value.dtype and out.shape == (value.shape[0], loc.shape[1], value.shape[2] * value.shape[3])
    assert gv.dtype == value.dtype and gl.dtype == loc.dtype and ga.dtype == attn.dtype
    ref = oracle.forward(value, shapes, starts, loc, attn, softmax=softmax)
    rgv, rgl, rga = oracle.backward(value, shapes, starts, loc, attn, grad_output, softmax=softmax)
    errs = {
        "output": rel_err(out, ref),
        "grad_value": rel_err(gv, rgv),
        "grad_loc": rel_err(gl, rgl),
        "grad_attn": rel_err(ga, rga.reshape(ga.shape)),
    }
    tols = {"output": FWD_TOL[dtype], "grad_value": BWD_TOL[dtype], "grad_loc": BWD_TOL[dtype],
            "grad_attn": BWD_TOL[dtype]}
    bad = {k: v for k, v in errs.items() if not v <= tols[k]}
    assert not bad, f"{label} softmax={softmax}: relative errors {errs} exceed {tols}"
    return errs


# BASELINE configurations 0-3 at full size (config 4 has its own test below).
CASES = [
    pytest.param(0, F32, F32, id="cfg0-f32"),
    pytest.param(1, F32, F32, id="cfg1-f32"),
    pytest.param(2, BF16, BF16, id="cfg2-bf16"),
    pytest.param(2, BF16, F32, id="cfg2-bf16-f32loc"),
    pytest.param(2, F16, F16, id="cfg2-f16"),
    pytest.param(3, F32, F32, id="cfg3-f32"),
    pytest.param(3, BF16, BF16, id="cfg3-bf16"),
]


@pytest.mark.parametrize("softmax", [False, True], ids=["linear", "softmax"])
@pytest.mark.parametrize(("cfg", "dtype", "loc_dtype"), CASES)
def test_baseline_configs_match_oracle(device, cfg, dtype, loc_dtype, softmax):
    w = make_workload(cfg).to(device, dtype, loc_dtype)
    check_against_oracle(*w.operands(softmax=softmax), w.grad_output, softmax=softmax, dtype=dtype,
                         label=f"config {cfg}")


@pytest.mark.slow
@pytest.mark.parametrize(("dtype", "loc_dtype"), [(BF16, BF16), (F16, F16), (BF16, F32)],
                         ids=["bf16", "f16", "bf16-f32loc"])
def test_headline_config_full_size_matches_oracle(device, dtype, loc_dtype):
    """Config 4 (B=4, Q=S=21,504, bf16) at full size, both methods."""
    w = make_workload(4).to(device, dtype, loc_dtype)
    for softmax in (False, True):
        check_against_oracle(*w.operands(softmax=softmax), w.grad_output, softmax=softmax, dtype=dtype,
                             label="config 4")


def test_headline_config_float32(device):
    w = make_workload(4, batch=1).to(device, F32)
    check_against_oracle(*w.operands(), w.grad_output, softmax=False, dtype=F32, label="config 4 f32")


# Shape coverage beyond the BASELINE configurations.

SHAPES = [
    # (levels, B, Q, H, D, P)
    pytest.param(((8, 8),), 1, 5, 1, 16, 4, id="one-level"),
    pytest.param(((8, 8), (4, 4), (2, 2)), 2, 12, 4, 32, 4, id="three-levels"),
    pytest.param(((7, 5), (3, 3)), 1, 9, 8, 16, 8, id="eight-points"),
    pytest.param(((1, 1),), 3, 4, 2, 16, 1, id="1x1-level"),
    pytest.param(((6, 9), (3, 5)), 2, 7, 3, 24, 3, id="odd-heads-d24-p3"),
    pytest.param(((6, 6), (3, 3)), 1, 10, 2, 8, 2, id="d8"),
    pytest.param(((9, 7), (5, 4)), 2, 33, 4, 64, 4, id="d64"),
    pytest.param(((9, 7),), 1, 17, 2, 128, 4, id="d128"),
    pytest.param(((5, 5),), 1, 6, 2, 7, 2, id="d7"),
    pytest.param(((10, 12), (5, 6), (3, 3), (2, 2), (1, 1)), 2, 21, 8, 32, 4, id="five-levels"),
    pytest.param(((12, 10), (6, 5)), 1, 13, 1, 256, 2, id="d256"),
    pytest.param(((11, 9), (6, 5), (3, 3)), 2, 19, 3, 48, 4, id="d48"),
    pytest.param(((9, 11), (5, 6), (3, 3), (2, 2)), 2, 25, 8, 32, 5, id="four-levels-p5"),
    pytest.param(((8, 8), (4, 4)), 1, 7, 3, 128, 6, id="d128-p6"),
    pytest.param(((7, 8), (4, 4)), 1, 11, 5, 16, 7, id="odd-heads-p7"),
    pytest.param(((10, 12), (5, 6), (3, 3), (2, 2), (1, 1)), 1, 9, 2, 64, 8, id="five-levels-p8"),
    # D = 8 with many samples: a unit takes more lanes than its channels need, so
    # that one wave's staging fits the LDS (found by the hypothesis sweep).
    pytest.param(((1, 1), (1, 1), (1, 1), (1, 1)), 1, 1, 1, 8, 7, id="d8-p7-tiny"),
    pytest.param(((9, 11), (5, 6), (3, 3), (2, 2), (1, 1)), 2, 37, 3, 8, 8, id="d8-five-levels-p8"),
]


@pytest.mark.parametrize("dtype", [F32, BF16, F16, F64], ids=["f32", "bf16", "f16", "f64"])
@pytest.mark.parametrize(("levels", "B", "Q", "H", "D", "P"), SHAPES)
def test_shapes_match_oracle(device, levels, B, Q, H, D, P, dtype):
    if dtype == F64 and D // 2 > 64:
        pytest.skip("float64 takes at most 64 lanes of 2 channels (D <= 128)")
    w = make_workload(0, levels=levels, batch=B, queries=Q, heads=H, channels=D, points=P, seed=Q + D)
    w = w.to(device, dtype)
    for softmax in (False, True):
        check_against_oracle(*w.operands(softmax=softmax), w.grad_output, softmax=softmax, dtype=dtype,
                             label=f"levels={levels} B={B} Q={Q} H={H} D={D} P={P}")


# Wider shapes at the size of an encoder (config 2's pyramid, Q = S = 5,376), where
# the bucket sort and the matrix-core grad_value kernel run as at full size:
# P not a multiple of 4 (per-sample bucketing), other head widths and head counts,
# and Deformable DETR's four levels.
WIDE = [
    pytest.param({"points": 3}, BF16, id="p3-bf16"),
    pytest.param({"points": 5}, F16, id="p5-f16"),
    pytest.param({"channels": 64, "heads": 4}, BF16, id="d64-h4-bf16"),
    pytest.param({"channels": 16, "heads": 5, "points": 8}, BF16, id="d16-h5-p8-bf16"),
    pytest.param({"channels": 48, "heads": 3}, F16, id="d48-h3-f16"),
    pytest.param({"levels": ((64, 64), (32, 32), (16, 16), (8, 8))}, BF16, id="four-levels-bf16"),
    pytest.param({"points": 6, "heads": 7}, F32, id="p6-h7-f32"),
]


@pytest.mark.parametrize(("sizes", "dtype"), WIDE)
def test_wider_shapes_at_encoder_size(device, sizes, dtype):
    w = make_workload(2, **sizes).to(device, dtype)
    for softmax in (False, True):
        check_against_oracle(*w.operands(softmax=softmax), w.grad_output, softmax=softmax, dtype=dtype,
                             label=f"config 2 with {sizes}")


# The two grad_value kernels for float and 16-bit dtypes: the matrix-core one (the
# default for D = 16, 32, 48, 64) and the VALU owner kernel (every other case, float64,
# and the fallback when the bucket scratch is short), forced by PATH_NO_MFMA; and the
# two ways the bucket sort publishes its counts: per-workgroup count rows (the default
# where the scratch has room) or global atomics, forced by PATH_ATOMIC_SORT; and the
# matrix-core kernel's 8 x 8 tiles at every level, forced by PATH_TILE8 (by default
# levels with few heavy tiles take 4 x 4 tiles: configs 2 and 3 both have such levels).

PATH_BITS = {"mfma": 0, "mfma-atomic-sort": 2, "mfma-tile8": 4, "valu": 1, "valu-atomic-sort": 3}


@pytest.mark.parametrize("path", sorted(PATH_BITS))
@pytest.mark.parametrize("dtype", [BF16, F16, F32], ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("cfg", [2, 3])
def test_grad_value_paths_match_oracle(device, cfg, dtype, path):
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    w = make_workload(cfg).to(device, dtype)
    with _lib.path_override(PATH_BITS[path]):
        for softmax in (False, True):
            check_against_oracle(*w.operands(softmax=softmax), w.grad_output, softmax=softmax, dtype=dtype,
                                 label=f"config {cfg} {path}")


@pytest.mark.parametrize(("dtype", "queries"), [(BF16, 256), (F32, 128)], ids=["bf16", "f32"])
def test_counters_that_do_not_fit_fall_back_to_the_owner_kernel(device, dtype, queries):
    """A 2 x 1024 level has 128 tiles of 8 x 8, where levels of aspect ratio up to 4
    would have about 49. With these queries the weight-gradient scratch holds 512
    counters per head: enough for the host's estimate, so the matrix-core kernel is
    launched, but not for the real counters plus its queue counters, so it does
    nothing and the VALU owner kernel launched after it computes grad_value."""
    w = make_workload(0, levels=((2, 1024),), batch=1, queries=queries, heads=2, channels=32, points=4,
                      seed=11).to(device, dtype)
    for softmax in (False, True):
        check_against_oracle(*w.operands(softmax=softmax), w.grad_output, softmax=softmax, dtype=dtype,
                             label=f"2x1024 level, {queries} queries")


@pytest.mark.parametrize("softmax", [False, True], ids=["linear", "softmax"])
@pytest.mark.parametrize(
    ("dtype", "cfg", "sizes"),
    [
        pytest.param(BF16, 2, {"queries": 1500}, id="bf16-matrix-cores"),
        pytest.param(F32, 2, {"queries": 1500}, id="f32-matrix-cores"),
        pytest.param(F32, 2, {"queries": 1500, "channels": 24, "points": 3}, id="f32-valu-per-sample-sort"),
        pytest.param(BF16, 1, {"batch": 2}, id="bf16-decoder-standby"),
    ],
)
def test_accumulate_flag_adds_into_grad_value(device, dtype, cfg, sizes, softmax):
    """MSDA_ACCUMULATE_GRAD_VALUE through the C ABI: grad_value = previous + gradient,
    with the other two gradients as without the flag."""
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    lib = _lib.load()
    w = make_workload(cfg, **{"batch": 1, **sizes}).to(device, dtype)
    value, shapes, starts, loc, attn = w.operands(softmax=softmax)
    method = _lib.FLAG_SOFTMAX if softmax else 0
    B, S, H, D, Q, L, P = w.sizes
    stream = torch.cuda.current_stream()
    codes = (_lib.DTYPE_CODES[value.dtype], _lib.DTYPE_CODES[loc.dtype], _lib.INDEX_CODES[shapes.dtype])

    def backward(grad_value, flags):
        gl, ga = torch.empty_like(loc), torch.empty_like(attn)
        lib.check(lib.backward(value.data_ptr(), codes[0], shapes.data_ptr(), starts.data_ptr(), codes[2],
                               loc.data_ptr(), codes[1], attn.data_ptr(), w.grad_output.data_ptr(),
                               grad_value.data_ptr(), gl.data_ptr(), ga.data_ptr(),
                               B, S, H, D, Q, L, P, flags, stream.cuda_stream))
        torch.cuda.synchronize()
        return grad_value, gl, ga

    plain = backward(torch.empty_like(value), method)
    previous = torch.randn(value.shape, generator=torch.Generator().manual_seed(3)).to(device, dtype)
    added = backward(previous.clone(), method | _lib.FLAG_ACCUMULATE_GRAD_VALUE)
    expected = previous.double() + plain[0].double()
    assert rel_err(added[0], expected.cpu()) <= BWD_TOL[dtype]
    torch.testing.assert_close(added[1], plain[1], rtol=0, atol=0)
    torch.testing.assert_close(added[2], plain[2], rtol=0, atol=0)


def abi_backward(w, flags, *, softmax=False, grad_value=None):
    """One backward C-ABI call on a workload; returns (grad_value, grad_loc, grad_attn)."""
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    lib = _lib.load()
    value, shapes, starts, loc, attn = w.operands(softmax=softmax)
    B, S, H, D, Q, L, P = w.sizes
    gv = torch.empty_like(value) if grad_value is None else grad_value
    gl, ga = torch.empty_like(loc), torch.empty_like(attn)
    flags |= _lib.FLAG_SOFTMAX if softmax else 0
    lib.check(lib.backward(value.data_ptr(), _lib.DTYPE_CODES[value.dtype], shapes.data_ptr(), starts.data_ptr(),
                           _lib.INDEX_CODES[shapes.dtype], loc.data_ptr(), _lib.DTYPE_CODES[loc.dtype],
                           attn.data_ptr(), w.grad_output.data_ptr(), gv.data_ptr(), gl.data_ptr(), ga.data_ptr(),
                           B, S, H, D, Q, L, P, flags, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return gv, gl, ga


@pytest.mark.parametrize("softmax", [False, True], ids=["linear", "softmax"])
@pytest.mark.parametrize(
    ("dtype", "sizes"),
    [
        pytest.param(F32, {}, id="f32"),
        pytest.param(F64, {}, id="f64"),
        pytest.param(BF16, {"queries": 100}, id="bf16"),
        pytest.param(F16, {"queries": 100}, id="f16"),
        pytest.param(BF16, {"queries": 100, "channels": 7}, id="bf16-one-channel-per-lane"),
        pytest.param(F16, {"queries": 100, "channels": 9, "heads": 3}, id="f16-one-channel-per-lane"),
    ],
)
def test_atomic_grad_value_flag_matches_oracle(device, dtype, sizes, softmax):
    """MSDA_GRAD_VALUE_ATOMIC: grad_value zero-filled, then scattered with global
    atomics in the value dtype (the reference's mechanism, include/interpolate.cuh:
    146-175). grad_value matches the oracle; the other two gradients are bit-equal to
    the default path's. 16-bit grad_value sums in its own dtype (one rounding per
    contribution), so those cases keep the coarsest level's fan-in near 100."""
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    w = make_workload(0, **sizes).to(device, dtype)
    value, shapes, starts, loc, attn = w.operands(softmax=softmax)
    atomic = abi_backward(w, _lib.FLAG_GRAD_VALUE_ATOMIC, softmax=softmax)
    owner = abi_backward(w, 0, softmax=softmax)
    expected = oracle.backward(value, shapes, starts, loc, attn, w.grad_output, softmax=softmax)[0]
    assert rel_err(atomic[0], expected) <= BWD_TOL[dtype]
    torch.testing.assert_close(atomic[1], owner[1], rtol=0, atol=0)
    torch.testing.assert_close(atomic[2], owner[2], rtol=0, atol=0)
    previous = torch.randn(value.shape, generator=torch.Generator().manual_seed(5)).to(device, dtype)
    added = abi_backward(w, _lib.FLAG_GRAD_VALUE_ATOMIC | _lib.FLAG_ACCUMULATE_GRAD_VALUE, softmax=softmax,
                         grad_value=previous.clone())[0]
    assert rel_err(added, (previous.double().cpu() + expected)) <= BWD_TOL[dtype]


@pytest.mark.parametrize("path", ["mfma", "valu"])
@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "f16"])
def test_weights_keep_fp32_precision(device, dtype, path):
    """The attention * bilinear weights stay fp32 in 16-bit calls, as in the reference
    (the fp32 acc of its Triton and CUDA kernels). Two queries sample the same two places
    (left, where value is +1, and right, where it is -1) at dx = 5/16, dy = 3/16 with
    attention weights a0 = 91/128 and a1 = 181/256 swapped between them, and grad_out
    is +1 for query 0 and -1 for query 1. Every product a * bilinear has 15
    significant bits, so rounding it to 16 bits (8 significant bits for bf16) would
    move the results by ~2^-9 a; the exact results are tiny by cancellation:
      output[q0] = a0 - a1 = 2^-8, output[q1] = -2^-8,
      grad_value = +-bilinear_c * 2^-8 at the corners of the left / right sample.
    All are representable, so fp32 weights give them exactly."""
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    W = Hh = 16
    D = 16
    value = torch.ones(1, Hh, W, 1, D, dtype=F64)
    value[:, :, W // 2:] = -1.0
    value = value.reshape(1, Hh * W, 1, D)
    x_left, x_right, y = 3 + 5 / 16, 11 + 5 / 16, 5 + 3 / 16
    # Queries past the first two have zero weight and gradient; they only give the
    # backward's sort enough scratch for the matrix-core kernel's counters.
    Q = 512
    loc = torch.tensor([(x_left + 0.5) / W, (y + 0.5) / Hh, (x_right + 0.5) / W, (y + 0.5) / Hh], dtype=F64)
    loc = loc.view(1, 1, 1, 1, 2, 2).expand(1, Q, 1, 1, 2, 2).contiguous()
    a0, a1 = 91 / 128, 181 / 256
    attn = torch.zeros(1, Q, 1, 2, dtype=F64)
    attn[0, :2, 0] = torch.tensor([[a0, a1], [a1, a0]], dtype=F64)
    grad_out = torch.zeros(1, Q, D, dtype=F64)
    grad_out[0, 0], grad_out[0, 1] = 1.0, -1.0
    shapes = torch.tensor([[Hh, W]])
    starts = torch.tensor([0])
    ops = [t.to(device, dtype) for t in (value, loc, attn, grad_out)]
    for t, ref in zip(ops, (value, loc, attn, grad_out)):
        assert torch.equal(t.double().cpu(), ref)  # the inputs are exact in the dtype
    with _lib.path_override(1 if path == "valu" else 0):
        out, gv, _, _ = run_hip(ops[0], shapes.to(device), starts.to(device), ops[1], ops[2], ops[3],
                                softmax=False)
    expected_out = oracle.forward(value, shapes, starts, loc, attn, softmax=False)
    expected_gv = oracle.backward(value, shapes, starts, loc, attn, grad_out, softmax=False)[0]
    assert expected_out.abs().max().item() == 2.0**-8
    torch.testing.assert_close(out.double().cpu(), expected_out.reshape(out.shape), rtol=0, atol=0)
    torch.testing.assert_close(gv.double().cpu(), expected_gv.reshape(gv.shape), rtol=0, atol=0)


@pytest.mark.parametrize(("cfg", "dtype"), [(2, BF16), (2, F16), (3, BF16), (4, BF16), (4, F16)])
def test_sixteen_bit_error_margin(device, cfg, dtype):
    """The measured norm-wise errors of 16-bit calls at configs 2-4 (config 4 at one
    image), printed, against a bound of two roundings to the value dtype (2^-8 for
    bf16, 2^-10 for f16): the result is one fp32 computation rounded once to the
    dtype, so it sits far inside the 2e-2 tolerance of the north star."""
    sizes = {"batch": 1} if cfg == 4 else {}
    w = make_workload(cfg, **sizes).to(device, dtype)
    bound = 2.0**-8 if dtype == BF16 else 2.0**-10
    for softmax in (False, True):
        errs = check_against_oracle(*w.operands(softmax=softmax), w.grad_output, softmax=softmax, dtype=dtype,
                                    label=f"config {cfg}")
        print(f"config {cfg} {dtype} softmax={softmax}: {errs}")
        assert max(errs.values()) <= bound, errs


@pytest.mark.parametrize("dtype", [BF16, F32], ids=["bf16", "f32"])
def test_grad_value_at_an_unaligned_offset(device, dtype):
    """A grad_value one element past its allocation's alignment (a caller's offset
    view): the grouped sort cannot park its 8- or 16-byte key words there, the
    matrix-core owner cannot store 16-byte rows and the sample kernel takes one
    channel per lane, so the call runs the per-sample sort and the VALU owner.
    Every gradient still matches the oracle."""
    w = make_workload(0, queries=200).to(device, dtype)
    value, shapes, starts, loc, attn = w.operands()
    flat = torch.empty(value.numel() + 1, dtype=dtype, device=device)
    shifted = flat[1:].view(value.shape)
    assert shifted.data_ptr() % 16 == value.element_size()
    gv, gl, ga = abi_backward(w, 0, grad_value=shifted)
    expected = oracle.backward(value, shapes, starts, loc, attn, w.grad_output, softmax=False)
    for got, want in zip((gv, gl, ga), expected):
        assert rel_err(got, want) <= BWD_TOL[dtype]


def test_atomic_grad_value_at_the_headline_loses_precision(device):
    """The reason the default backward does not scatter grad_value with atomics, at
    config 4 (one image): 16-bit atomics round every contribution into a 16-bit
    sum (fan-in up to ~1,300 at the coarsest level), where the owners sum in fp32
    and round once. Measured: norm-wise error against the oracle and the
    directional bias |cos(mean error, gradient)| of grad_value (grad_out = 1, the
    reference's tests/deformops/test_msda_bias.py), both paths, bf16 and fp32."""
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    base = make_workload(4, batch=1)
    base.grad_output = torch.ones_like(base.grad_output)
    value, shapes, starts, loc, attn = base.operands()
    exact = oracle.backward(value, shapes, starts, loc, attn, base.grad_output, softmax=False)[0]
    found = {}
    for dtype in (BF16, F32):
        w = base.to(device, dtype)
        rounded = [t.double().cpu() for t in (w.value, w.sampling_locations, w.attention_weights)]
        expected = oracle.backward(rounded[0], shapes, starts, rounded[1], rounded[2], base.grad_output,
                                   softmax=False)[0]
        for name, flags in (("owner", 0), ("atomic", _lib.FLAG_GRAD_VALUE_ATOMIC)):
            gv = abi_backward(w, flags)[0].double().cpu()
            err = gv - expected
            cos = (err * exact).sum().item() / (err.norm().item() * exact.norm().item() + 1e-30)
            found[(dtype, name)] = (rel_err(gv, expected), cos)
    print("config 4, one image, grad_value (norm-wise error, bias cos):",
          {f"{str(d).split('.')[-1]} {n}": (f"{e:.2e}", f"{c:+.3f}") for (d, n), (e, c) in found.items()})
    assert found[(BF16, "owner")][0] <= 2.0**-8
    assert found[(BF16, "atomic")][0] > 4 * found[(BF16, "owner")][0]
    assert found[(F32, "owner")][0] <= BWD_TOL[F32] and found[(F32, "atomic")][0] <= BWD_TOL[F32]


# Overlapping level tables: two valid levels that share positions of S. The forward
# samples each level as given; the backward sums every level's contribution into a
# shared grad_value element, as the oracle and the reference's eager path do (its
# flat indices start + y W + x, backends/eager/msda_pytorch.py:83-112, under autograd).
OVERLAPS = [
    # (levels, starts, S): level 1 starts inside level 0
    pytest.param(((6, 5), (4, 4)), (0, 10), 30, id="second-inside-first"),
    # identical levels, both at 0
    pytest.param(((5, 5), (5, 5)), (0, 0), 25, id="same-level-twice"),
    # three levels, the last overlapping the first two
    pytest.param(((8, 8), (4, 4), (6, 6)), (0, 64, 50), 86, id="third-spans-two"),
]


@pytest.mark.parametrize("path", ["default", "valu"])
@pytest.mark.parametrize("dtype", [F32, BF16, F64], ids=["f32", "bf16", "f64"])
@pytest.mark.parametrize(("levels", "starts", "S"), OVERLAPS)
def test_overlapping_levels_sum_into_grad_value(device, levels, starts, S, dtype, path):
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    L = len(levels)
    g = torch.Generator().manual_seed(17)
    B, Q, H, D, P = 2, 30, 2, 16, 4
    value = torch.randn(B, S, H, D, generator=g, dtype=F64)
    loc = torch.rand(B, Q, H, L, P, 2, generator=g, dtype=F64) * 1.1 - 0.05
    attn = torch.softmax(torch.randn(B, Q, H, L * P, generator=g, dtype=F64), -1)
    grad_out = torch.randn(B, Q, H * D, generator=g, dtype=F64)
    shapes = torch.tensor(levels, dtype=torch.int64)
    start_t = torch.tensor(starts, dtype=torch.int64)
    ops = [t.to(device, dtype) for t in (value, loc, attn, grad_out)]
    with _lib.path_override(1 if path == "valu" else 0):
        for softmax in (False, True):
            check_against_oracle(ops[0], shapes.to(device), start_t.to(device), ops[1], ops[2], ops[3],
                                 softmax=softmax, dtype=dtype, label=f"overlap {levels} {starts} {path}")


def abi_backward_into(lib, w, grads, flags, stream, workspace=None):
    """One msda_backward call (workspace None) or msda_backward_workspace call on the
    workload's operands, writing into ``grads`` = (grad_value, grad_loc, grad_attn)."""
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    value, shapes, starts, loc, attn = w.operands(softmax=bool(flags & _lib.FLAG_SOFTMAX))
    B, S, H, D, Q, L, P = w.sizes
    args = (value.data_ptr(), _lib.DTYPE_CODES[value.dtype], shapes.data_ptr(), starts.data_ptr(),
            _lib.INDEX_CODES[shapes.dtype], loc.data_ptr(), _lib.DTYPE_CODES[loc.dtype], attn.data_ptr(),
            w.grad_output.data_ptr(), *(t.data_ptr() for t in grads), B, S, H, D, Q, L, P, flags)
    if workspace is None:
        lib.check(lib.backward(*args, stream))
    else:
        lib.check(lib.backward_workspace(*args, workspace.data_ptr(), workspace.numel(), stream))


def workspace_for(lib, w, flags=0):
    value = w.value
    size = lib.workspace_size(value.dtype, *w.sizes, flags)
    return torch.empty(size, dtype=torch.uint8, device=value.device)


@pytest.mark.parametrize("softmax", [False, True], ids=["linear", "softmax"])
@pytest.mark.parametrize(("cfg", "dtype", "batch", "queries"),
                         [(4, BF16, None, None), (2, F16, 1, 3000), (3, F32, None, None), (1, F32, None, None)],
                         ids=["cfg4-bf16", "cfg2-f16", "cfg3-f32", "cfg1-f32"])
def test_workspace_backward_matches_the_plain_backward(device, cfg, dtype, batch, queries, softmax):
    """msda_backward_workspace runs grad_sample beside the sort on a side stream: its
    location and weight gradients are the same kernel's on the same inputs (bit-equal),
    grad_value the same sums in another order. A workspace one byte short, or
    misaligned, gives the plain call's schedule with the same results."""
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    lib = _lib.load()
    kwargs = {k: v for k, v in (("batch", batch), ("queries", queries)) if v is not None}
    w = make_workload(cfg, **kwargs).to(device, dtype)
    flags = _lib.FLAG_SOFTMAX if softmax else 0
    st = torch.cuda.current_stream().cuda_stream
    plain = [torch.empty_like(t) for t in (w.value, w.sampling_locations, w.attention_weights)]
    abi_backward_into(lib, w, plain, flags, st)
    size = lib.workspace_size(w.value.dtype, *w.sizes, flags)
    ws = torch.empty(size + 64, dtype=torch.uint8, device=device)  # 512-byte aligned base
    for workspace in (ws[:size], ws[: size - 1], ws[64:]):
        got = [torch.full_like(t, float("nan")) for t in plain]
        ws.fill_(255)  # the workspace's contents must not matter
        abi_backward_into(lib, w, got, flags, st, workspace=workspace)
        torch.cuda.synchronize()
        assert rel_err(got[0], plain[0].double().cpu()) <= BWD_TOL[dtype]
        torch.testing.assert_close(got[1], plain[1], rtol=0, atol=0)
        torch.testing.assert_close(got[2], plain[2], rtol=0, atol=0)


@pytest.mark.parametrize("dtype", [BF16, F32], ids=["bf16", "f32"])
def test_small_sort_counts_in_its_scratch_row_when_lds_is_short(device, dtype):
    """A call of few samples per (b, h) sorts in one launch, its bucket counters in
    LDS. A 1024 x 1024 level has 16,384 tiles of 8 x 8, 65,536 counters, more than
    the 160 KB of LDS hold, so the kernel counts in its own row of the workspace's
    scratch instead (the autograd bridge passes a workspace that holds them)."""
    w = make_workload(1, batch=1, queries=60, heads=2, channels=16, levels=((1024, 1024),), locations="uniform")
    w = w.to(device, dtype)
    for softmax in (False, True):
        check_against_oracle(*w.operands(softmax=softmax), w.grad_output, softmax=softmax, dtype=dtype,
                             label="one 1024 x 1024 level")


def test_many_images_keep_one_queue_mode(device):
    """The matrix-core grad_value kernel deals (image, region) pairs to eight XCD
    queues. With 8,193 images of one 8 x 8 level (one region each) the queues get
    1,024 or 1,025 pairs, around the 1,024 entries a queue's LDS table holds: every
    queue must then take the same mode (here the raster split of each level's tasks),
    or tasks would be done twice and others never (with two heads the two splits
    differ: image 7,168's first head belonged to neither)."""
    w = make_workload(0, batch=8193, queries=1, heads=2, channels=16, levels=((8, 8),), locations="uniform")
    w = w.to(device, BF16)
    check_against_oracle(*w.operands(), w.grad_output, softmax=False, dtype=BF16, label="8193 images")


@pytest.mark.parametrize("entry", ["plain", "workspace"])
@pytest.mark.parametrize("dtype", [BF16, F32], ids=["bf16", "f32"])
def test_calls_replay_from_a_hip_graph(device, dtype, entry):
    """The forward and backward C-ABI calls launch kernels only (no allocation, no
    memset), so a caller can capture them in a HIP graph; the workspace backward's
    fork onto its side stream and join back are captured as graph edges. Each
    replay, with eager work in between that poisons the outputs, must give the
    eager results."""
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    lib = _lib.load()
    # The workspace entry forks grad_sample onto its side stream from 2^21 samples:
    # config 2's pyramid over 5 images (2.6 M samples) does; the plain entry takes a
    # smaller call.
    w = (make_workload(2, batch=5) if entry == "workspace" else make_workload(2, batch=1, queries=2000))
    w = w.to(device, dtype)
    value, shapes, starts, loc, attn = w.operands(softmax=True)
    B, S, H, D, Q, L, P = w.sizes
    codes = (_lib.DTYPE_CODES[value.dtype], _lib.DTYPE_CODES[loc.dtype], _lib.INDEX_CODES[shapes.dtype])
    out = torch.empty((B, Q, H * D), dtype=dtype, device=device)
    gv, gl, ga = torch.empty_like(value), torch.empty_like(loc), torch.empty_like(attn)
    ws = workspace_for(lib, w, _lib.FLAG_SOFTMAX) if entry == "workspace" else None

    def calls() -> None:
        st = torch.cuda.current_stream().cuda_stream
        lib.check(lib.forward(value.data_ptr(), codes[0], shapes.data_ptr(), starts.data_ptr(), codes[2],
                              loc.data_ptr(), codes[1], attn.data_ptr(), out.data_ptr(),
                              B, S, H, D, Q, L, P, _lib.FLAG_SOFTMAX, st))
        abi_backward_into(lib, w, (gv, gl, ga), _lib.FLAG_SOFTMAX, st, workspace=ws)

    calls()
    torch.cuda.synchronize()
    eager = [t.clone() for t in (out, gv, gl, ga)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        calls()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        calls()
    for _ in range(3):
        for t in (out, gv, gl, ga):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        if ws is not None:
            ws.fill_(255)
        for got, want in zip((out, gv, gl, ga), eager):
            assert not torch.isnan(got).any()
            # grad_value's summation order may differ between runs; the rest is exact.
            tol = BWD_TOL[dtype] if got is gv else 0.0
            assert rel_err(got, want.double().cpu()) <= tol


@pytest.mark.parametrize("entry", ["plain", "workspace"])
def test_concurrent_calls_from_two_threads_on_two_streams(device, entry):
    """The library keeps no state between calls (scratch lives in each call's outputs
    or workspace, side streams and errors are per thread): two host threads, each
    calling the backward on its own stream with its own workload, get the sequential
    results."""
    import threading  # noqa: PLC0415

    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    lib = _lib.load()
    # Config 2's pyramid over 5 images (2.6 M samples) for the workspace entry, so that
    # each thread forks onto a side stream of its own.
    sizes = {"batch": 5} if entry == "workspace" else {"batch": 1, "queries": 1800}
    works = [make_workload(2, seed=s, **sizes).to(device, dt) for s, dt in ((1, BF16), (2, F32))]

    def backward(w, stream):
        grads = [torch.empty_like(t) for t in (w.value, w.sampling_locations, w.attention_weights)]
        ws = workspace_for(lib, w) if entry == "workspace" else None
        abi_backward_into(lib, w, grads, 0, stream.cuda_stream, workspace=ws)
        return grads

    stream0 = torch.cuda.current_stream()
    expected = [backward(w, stream0) for w in works]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    results: list = [None, None]
    errors: list = []

    def run(i):
        try:
            with torch.cuda.stream(streams[i]):
                results[i] = [backward(works[i], streams[i]) for _ in range(4)]
        except Exception as exc:  # noqa: BLE001 - reported below
            errors.append(exc)

    threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for i, w in enumerate(works):
        dt = w.value.dtype
        for gv, gl, ga in results[i]:
            assert rel_err(gv, expected[i][0].double().cpu()) <= BWD_TOL[dt]
            torch.testing.assert_close(gl, expected[i][1], rtol=0, atol=0)
            torch.testing.assert_close(ga, expected[i][2], rtol=0, atol=0)


@pytest.mark.parametrize("dtype", [BF16, F16, F32], ids=["bf16", "f16", "f32"])
def test_samples_piled_on_one_tile(device, dtype):
    """Every sample of every query lands near one pixel: one tile owns them all, so a
    tile runs many K-blocks per wave and its neighbours get only straddlers."""
    g = torch.Generator().manual_seed(9)
    w = make_workload(0, levels=((24, 20), (12, 10)), batch=2, queries=700, heads=2, channels=32, points=4)
    B, S, H, D, Q, L, P = w.sizes
    centre = torch.tensor([0.41, 0.57], dtype=torch.float64)
    loc = centre + 0.01 * torch.randn(B, Q, H, L, P, 2, generator=g, dtype=torch.float64)
    w = dataclasses.replace(w, sampling_locations=loc.to(w.sampling_locations.dtype)).to(device, dtype)
    for softmax in (False, True):
        check_against_oracle(*w.operands(softmax=softmax), w.grad_output, softmax=softmax, dtype=dtype,
                             label="piled")


# Boundary semantics.


def test_pixel_boundary_table_matches_grid_sample(device):
    """Exact pixel transitions (reference tests/deformops/test_msda_eager.py:54-80)."""
    W = H = 4
    shapes = torch.tensor([[H, W]], device=device)
    starts = torch.tensor([0], device=device)
    value = torch.arange(H * W, dtype=F32, device=device).view(1, H * W, 1, 1)
    coords = [0.0, 0.125, 0.375, 0.5, 1.0, -0.125, 1.25]
    pts = [(cx, cy) for cx in coords for cy in coords]
    loc = torch.tensor(pts, dtype=F32, device=device).view(1, 1, 1, 1, len(pts), 2)
    attn = torch.ones(1, 1, 1, len(pts), dtype=F32, device=device)
    # One point per call, so each sample's value is visible on its own.
    for i in range(len(pts)):
        out = msda(value, shapes, starts, loc[..., i : i + 1, :], attn[..., i : i + 1])
        ref = grid_sample_msda(value.cpu(), shapes.cpu(), loc[..., i : i + 1, :].cpu(), attn[..., i : i + 1].cpu())
        torch.testing.assert_close(out.cpu(), ref, atol=1e-6, rtol=1e-6, msg=f"point {pts[i]}")


@pytest.mark.parametrize("softmax", [False, True], ids=["linear", "softmax"])
def test_grid_aligned_locations_match_eager_gradients(device, softmax):
    """Samples on integer pixels, -1 and the far edge included: one-sided gradients as
    eager autograd gives them (reference tests/deformops/test_release_regressions.py:264-339)."""
    g = torch.Generator().manual_seed(5)
    levels = ((8, 8), (4, 4), (2, 2))
    shapes = torch.tensor(levels)
    areas = shapes.prod(1)
    starts = torch.cat([areas.new_zeros(1), areas.cumsum(0)[:-1]])
    B, Q, H, D, P = 2, 11, 4, 8, 4
    value = torch.randn(B, int(areas.sum()), H, D, generator=g)
    pixels = torch.randint(-2, 10, (B, Q, H, len(levels), P, 2), generator=g).float()
    loc = (pixels + 0.5) / shapes.flip(1).view(1, 1, 1, -1, 1, 2)
    attn = torch.randn(B, Q, H, len(levels) * P, generator=g)
    grad = torch.linspace(-1, 1, B * Q * H * D).view(B, Q, H * D)

    leaves = [t.clone().requires_grad_(True) for t in (value, loc, attn)]
    expected = eager_msda(leaves[0], shapes, starts, leaves[1], leaves[2], softmax=softmax)
    expected.backward(grad)
    out, gv, gl, ga = run_hip(value.to(device), shapes.to(device), starts.to(device), loc.to(device),
                              attn.to(device), grad.to(device), softmax=softmax)
    for name, actual, ref in (("output", out, expected.detach()), ("value", gv, leaves[0].grad),
                              ("location", gl, leaves[1].grad), ("attention", ga, leaves[2].grad)):
        torch.testing.assert_close(actual.cpu(), ref, rtol=1e-4, atol=1e-5, msg=f"{name} differs")


def test_all_out_of_bounds_is_zero(device):
    w = make_workload(0, levels=((4, 4),), batch=1, queries=6, heads=2, channels=16).to(device, F32)
    loc = torch.full_like(w.sampling_locations, 5.0)
    out, gv, gl, ga = run_hip(w.value, w.spatial_shapes, w.level_start_index, loc, w.attention_weights,
                              w.grad_output, softmax=False)
    for t in (out, gv, gl, ga):
        assert torch.count_nonzero(t) == 0


@pytest.mark.parametrize("bad", [math.inf, -math.inf, math.nan])
def test_nonfinite_locations_contribute_nothing(device, bad):
    """A non-finite location is skipped: finite output and grad_value everywhere, the
    other queries unchanged (reference tests/deformops/test_msda_backward_robustness.py)."""
    w = make_workload(0, levels=((8, 8), (4, 4)), batch=2, queries=9, heads=2, channels=16).to(device, F32)
    loc = w.sampling_locations.clone()
    loc[:, 3] = bad
    out, gv, gl, ga = run_hip(w.value, w.spatial_shapes, w.level_start_index, loc, w.attention_weights,
                              w.grad_output, softmax=False)
    assert torch.isfinite(out).all() and torch.isfinite(gv).all()
    assert torch.count_nonzero(out[:, 3]) == 0
    keep = [q for q in range(loc.shape[1]) if q != 3]
    ref = oracle.forward(w.value, w.spatial_shapes, w.level_start_index, loc, w.attention_weights)
    assert rel_err(out[:, keep], ref[:, keep]) <= 1e-5
    rgv, rgl, _ = oracle.backward(w.value, w.spatial_shapes, w.level_start_index, loc, w.attention_weights,
                                  w.grad_output)
    assert rel_err(gv, rgv) <= 1e-4
    assert rel_err(gl[:, keep], rgl[:, keep]) <= 1e-4


def test_softmax_with_negative_infinite_logit(device):
    """A -inf logit gets zero weight; the rest of the softmax is unaffected."""
    w = make_workload(0, levels=((8, 8), (4, 4)), batch=1, queries=5, heads=2, channels=16).to(device, F32)
    logits = w.logits.clone()
    logits[..., 0] = -math.inf
    out, *_ = run_hip(w.value, w.spatial_shapes, w.level_start_index, w.sampling_locations, logits,
                      w.grad_output, softmax=True)
    ref = oracle.forward(w.value, w.spatial_shapes, w.level_start_index, w.sampling_locations, logits,
                         softmax=True)
    assert rel_err(out, ref) <= 1e-5


# Operand handling.


@pytest.mark.parametrize("axis", ["batch", "queries"])
def test_empty_calls(device, axis):
    sizes = {"batch": 0} if axis == "batch" else {"queries": 0}
    w = make_workload(0, levels=((4, 4),), heads=2, channels=16, **{"batch": 1, "queries": 3, **sizes})
    w = w.to(device, F32)
    out, gv, gl, ga = run_hip(w.value, w.spatial_shapes, w.level_start_index, w.sampling_locations,
                              w.attention_weights, w.grad_output, softmax=False)
    assert out.shape == (w.value.shape[0], w.sampling_locations.shape[1], 32)
    assert gv.shape == w.value.shape and torch.count_nonzero(gv) == 0


@pytest.mark.parametrize("method", ["linear", "softmax"])
def test_non_contiguous_operands(device, method):
    """Views with odd strides give the contiguous result and route gradients to the
    leaves (reference tests/deformops/test_release_regressions.py:154-214)."""
    w = make_workload(0, levels=((8, 8), (4, 4)), batch=2, queries=10, heads=2, channels=16).to(device, F32)
    value_leaf = w.value.transpose(1, 2).contiguous().requires_grad_(True)
    packed = torch.cat([w.sampling_locations, torch.rand_like(w.sampling_locations)], -1).requires_grad_(True)
    weights = w.logits if method == "softmax" else w.attention_weights
    attn_packed = torch.cat([weights, torch.rand_like(weights)], -1).requires_grad_(True)
    out = msda(value_leaf.transpose(1, 2), w.spatial_shapes, w.level_start_index, packed[..., :2],
               attn_packed[..., : weights.shape[-1]], method=method)
    out.backward(w.grad_output)
    ref_out, gv, gl, ga = run_hip(w.value, w.spatial_shapes, w.level_start_index, w.sampling_locations,
                                  weights, w.grad_output, softmax=method == "softmax")
    close = {"rtol": 1e-5, "atol": 1e-6}
    torch.testing.assert_close(out.detach(), ref_out, **close)
    torch.testing.assert_close(value_leaf.grad.transpose(1, 2), gv, **close)
    torch.testing.assert_close(packed.grad[..., :2], gl, **close)
    assert torch.count_nonzero(packed.grad[..., 2:]) == 0
    torch.testing.assert_close(attn_packed.grad[..., : weights.shape[-1]], ga, **close)
    assert torch.count_nonzero(attn_packed.grad[..., weights.shape[-1] :]) == 0


def test_split_weights_and_int32_tables(device):
    w = make_workload(0, levels=((8, 8), (4, 4)), batch=2, queries=7, heads=4, channels=32).to(device, F32)
    B, S, H, D, Q, L, P = w.sizes
    flat, *_ = run_hip(w.value, w.spatial_shapes, w.level_start_index, w.sampling_locations,
                       w.attention_weights, w.grad_output, softmax=True)
    split_w = w.attention_weights.view(B, Q, H, L, P)
    split, _, _, ga = run_hip(w.value, w.spatial_shapes.int(), w.level_start_index.int(),
                              w.sampling_locations, split_w, w.grad_output, softmax=True)
    assert ga.shape == (B, Q, H, L, P)
    torch.testing.assert_close(flat, split, rtol=0, atol=0)


def test_softmax_equals_linear_on_normalized_weights(device):
    """method="softmax" on logits equals "linear" on their softmax
    (reference tests/deformops/test_msda_cpu_fallbacks.py:19-37)."""
    w = make_workload(2, batch=1).to(device, F32)
    a, *_ = run_hip(*w.operands(softmax=True), w.grad_output, softmax=True)
    b, *_ = run_hip(w.value, w.spatial_shapes, w.level_start_index, w.sampling_locations,
                    torch.softmax(w.logits, -1), w.grad_output, softmax=False)
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("softmax", [False, True], ids=["linear", "softmax"])
def test_float64_gradcheck(device, softmax):
    """Finite-difference gradcheck in float64 (reference tests/deformops/test_msda_gradcheck.py)."""
    w = make_workload(0, levels=((5, 6), (3, 2)), batch=1, queries=3, heads=2, channels=4, points=2,
                      seed=11)
    w = w.to(device, F64)
    value, shapes, starts, loc, attn = w.operands(softmax=softmax)
    # Keep samples away from pixel boundaries, where the location gradient is one-sided.
    loc = (loc * 0.9 + 0.05).detach()

    def fn(v, l, a):  # noqa: E741
        return msda(v, shapes, starts, l, a, method="softmax" if softmax else "linear")

    inputs = tuple(t.detach().clone().requires_grad_(True) for t in (value, loc, attn))
    assert torch.autograd.gradcheck(fn, inputs, eps=1e-6, atol=1e-5, nondet_tol=1e-12)


# Dispatch surface.


def test_backend_selection_and_aliases(device):
    w = make_workload(0, levels=((8, 8),), batch=1, queries=4, heads=2, channels=16).to(device, F32)
    ops = w.operands()
    auto = msda(*ops)
    for backend in (Backend.HIP, Backend.CUDA):
        torch.testing.assert_close(msda(*ops, backend=backend), auto, rtol=0, atol=0)
    torch.testing.assert_close(torch.ops.deformops.msda(*ops), auto, rtol=0, atol=0)
    torch.testing.assert_close(
        torch.ops.deformops.msda_softmax(*w.operands(softmax=True)), msda(*w.operands(softmax=True), softmax=True)
    )
    with pytest.raises(NoBackendError, match="not part of this build"):
        msda(*ops, backend=Backend.TRITON)
    # The CPU backend takes CPU tensors only: never GPU ones, even when asked.
    with pytest.raises(NoBackendError, match="does not support"):
        msda(*ops, backend=Backend.EAGER)
    torch.testing.assert_close(msda(*(t.cpu() for t in ops)), auto.cpu(), rtol=1e-5, atol=1e-6)


def test_unsupported_head_dim_raises_no_backend_error(device):
    w = make_workload(0, levels=((4, 4),), batch=1, queries=2, heads=1, channels=1030).to(device, F32)
    with pytest.raises(NoBackendError, match="does not support"):
        msda(*w.operands(), backend=Backend.HIP)


def test_malformed_operands_raise_value_error(device):
    w = make_workload(0, levels=((4, 4), (2, 2)), batch=1, queries=8, heads=2, channels=16).to(device, F32)
    value, shapes, starts, loc, attn = w.operands()
    for bad in (
        (value, shapes, starts, torch.rand(*loc.shape[:-1], 3, device=device), attn),
        (value, shapes, starts, loc, attn[..., :-1]),
        (value, shapes, starts, loc, attn.half()),
    ):
        with pytest.raises(ValueError):  # noqa: PT011
            msda(*bad, backend=Backend.HIP)


def test_malformed_level_table_reads_nothing_out_of_bounds(device):
    """A level table that overruns value samples nothing from the bad level."""
    w = make_workload(0, levels=((8, 8), (4, 4)), batch=1, queries=6, heads=2, channels=16).to(device, F32)
    bad_shapes = torch.tensor([[8, 8], [40, 40]], device=device)
    out = msda(w.value, bad_shapes, w.level_start_index, w.sampling_locations, w.attention_weights)
    keep = w.sampling_locations.clone()
    ref_w = w.attention_weights.view(1, 6, 2, 2, 4).clone()
    ref_w[:, :, :, 1] = 0
    ref = oracle.forward(w.value, w.spatial_shapes, w.level_start_index, keep, ref_w.view(1, 6, 2, 8))
    assert rel_err(out, ref) <= 1e-5


@pytest.mark.parametrize("dtype", [BF16, F16, F32], ids=["bf16", "f16", "f32"])
def test_positions_outside_every_level_get_zero_gradient(device, dtype):
    """value rows that no level covers (a gap between the levels and a tail) get
    exactly zero in grad_value, which the kernels allocate uninitialized."""
    w = make_workload(0, levels=((8, 8), (4, 4)), batch=2, queries=30, heads=2, channels=32)
    B, S, H, D, Q, L, P = w.sizes
    starts = torch.tensor([0, 70])
    value = torch.randn(B, 90, H, D, generator=torch.Generator().manual_seed(5), dtype=torch.float64)
    w = dataclasses.replace(w, value=value, level_start_index=starts).to(device, dtype)
    for softmax in (False, True):
        check_against_oracle(*w.operands(softmax=softmax), w.grad_output, softmax=softmax, dtype=dtype,
                             label="gaps")
        _, gv, _, _ = run_hip(*w.operands(softmax=softmax), w.grad_output, softmax=softmax)
        assert torch.count_nonzero(gv[:, 64:70]) == 0 and torch.count_nonzero(gv[:, 86:]) == 0


# Precision of the 16-bit gradients: fp32 sums rounded once, so no drift.


@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "f16"])
def test_grad_value_is_unbiased(device, dtype):
    """|cos(mean error, fp64 gradient)| < 0.05 over 4 runs
    (reference tests/deformops/test_msda_bias.py:23-109)."""
    levels = ((48, 48), (24, 24), (12, 12))
    w = make_workload(0, levels=levels, batch=2, queries=1024, heads=8, channels=32, seed=1958)
    loc = w.sampling_locations * 0.8 + 0.1
    ones = torch.ones_like(w.grad_output)
    gt, _, _ = oracle.backward(w.value, w.spatial_shapes, w.level_start_index, loc, w.logits, ones,
                               softmax=True, pixel_f32=False)
    errors = []
    for _ in range(4):
        _, gv, _, _ = run_hip(w.value.to(device, dtype), w.spatial_shapes.to(device),
                              w.level_start_index.to(device), loc.to(device, dtype), w.logits.to(device, dtype),
                              ones.to(device, dtype), softmax=True)
        errors.append(gv.double().cpu() - gt)
    mean_err = torch.stack(errors).mean(0)
    cos = (mean_err * gt).sum().item() / (mean_err.norm().item() * gt.norm().item() + 1e-30)
    assert abs(cos) < 0.05, f"directional grad_value bias cos={cos:+.3f}"


# Second derivatives, non-finite weights on skipped samples, float32 product error.


@pytest.mark.parametrize("route", ["eager", "registered-op"])
def test_second_derivative_raises(device, route):
    """The kernels' gradients carry no graph, so a double backward must raise rather
    than come back as zeros: the backward is once-differentiable, as the reference
    CUDA bridge's (backends/cuda/_msda_bridge.py:232). Both routes: the plain-eager
    autograd.Function and the private operator's registered autograd."""
    w = make_workload(0, batch=1, queries=40, heads=2, channels=16).to(device, F32)
    value, shapes, starts, loc, attn = w.operands()
    leaves = [t.detach().clone().requires_grad_(True) for t in (value, loc, attn)]
    if route == "eager":
        out = msda(leaves[0], shapes, starts, leaves[1], leaves[2])
    else:
        out = torch.ops.deformops_hip.msda_forward(leaves[0], shapes, starts, leaves[1], leaves[2],
                                                   128, loc.shape[4], 0, 0)
    # A loss whose gradient with respect to the output depends on the leaves (as in a
    # gradient penalty): the once-differentiable guard wraps the gradients.
    # (.backward() runs every node of the graph; torch.autograd.grad with
    # allow_unused=True would prune the guard and return None instead.)
    grads = torch.autograd.grad(out.square().sum(), leaves, create_graph=True)
    assert all(g is not None and g.requires_grad for g in grads)
    with pytest.raises(RuntimeError, match="differentiate twice"):
        sum(g.square().sum() for g in grads).backward()
    # With a constant output gradient the kernels' gradients carry no graph at all,
    # and a second derivative raises too.
    grads = torch.autograd.grad((out * w.grad_output).sum(), leaves, create_graph=True)
    with pytest.raises(RuntimeError):
        sum(g.square().sum() for g in grads).backward()


@pytest.mark.parametrize("flags", ["default", "atomic"])
@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_infinite_weight_on_a_skipped_sample(device, dtype, flags):
    """A sample outside its level is skipped by the reference, whatever its weight: an
    infinite attention weight there must not turn its clamped corners' contributions
    into 0 * inf = NaN. The output and every gradient match the oracle run with that
    weight set to zero; the sample's own location and weight gradients are exactly
    zero. Run on the default backward and on the atomic scatter."""
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    w = make_workload(0, batch=1, queries=60, heads=2, channels=16)
    loc = w.sampling_locations.clone()
    attn = w.attention_weights.clone()
    loc[0, 7, 1, 0, 2] = torch.tensor([1.5, 0.5], dtype=loc.dtype)  # right of level 0
    attn[0, 7, 1, 2] = math.inf
    finite = attn.clone()
    finite[0, 7, 1, 2] = 0.0
    w = dataclasses.replace(w, sampling_locations=loc, attention_weights=attn).to(device, dtype)
    value, shapes, starts, _, _ = w.operands()
    ref_out = oracle.forward(value, shapes, starts, w.sampling_locations, finite.to(dtype))
    ref = oracle.backward(value, shapes, starts, w.sampling_locations, finite.to(dtype), w.grad_output)
    if flags == "default":
        out = run_hip(value, shapes, starts, w.sampling_locations, w.attention_weights, w.grad_output,
                      softmax=False)
        assert rel_err(out[0], ref_out) <= FWD_TOL[dtype]
        grads = out[1:]
    else:
        grads = abi_backward(w, _lib.FLAG_GRAD_VALUE_ATOMIC)
    for got, want in zip(grads, ref):
        assert torch.isfinite(got).all()
        assert rel_err(got, want) <= BWD_TOL[dtype]
    assert torch.count_nonzero(grads[1][0, 7, 1, 0, 2]) == 0
    assert grads[2][0, 7, 1, 2].item() == 0.0


@pytest.mark.parametrize("path", ["mfma", "valu"])
def test_float32_grad_value_elementwise_bound(device, path):
    """Float32 grad_value on the matrix cores multiplies bf16 parts of W and grad_out
    (W_hi G_hi + W_lo G_hi + W_hi G_lo), which bounds each product's relative error by
    3 * 2^-16; the sums are fp32. So every element, however much its contributions
    cancel, is within 4 * 2^-16 of sum_k |W_k G_k| (3 for the products, one for fp32
    accumulation over this fan-in) of the float64 result. The VALU owner multiplies
    in fp32 and stays within 2^-16. sum |W G| is the oracle's grad_value with |weights|
    and |grad_out| (the bilinear weights are non-negative)."""
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    w = make_workload(2, batch=1, queries=3000).to(device, F32)
    value, shapes, starts, loc, attn = w.operands()
    with _lib.path_override(1 if path == "valu" else 0):
        _, gv, _, _ = run_hip(value, shapes, starts, loc, attn, w.grad_output, softmax=False)
    exact = oracle.backward(value, shapes, starts, loc, attn, w.grad_output, softmax=False)[0]
    scale = oracle.backward(value, shapes, starts, loc, attn.abs(), w.grad_output.abs(), softmax=False)[0]
    err = (gv.double().cpu().reshape(exact.shape) - exact).abs()
    bound = (4.0 if path == "mfma" else 1.0) * 2.0**-16
    ratio = (err / scale.clamp_min(1e-30)).max().item()
    cancel = (exact.abs() / scale.clamp_min(1e-30))
    print(f"{path}: max err / sum|WG| = {ratio:.3e} (2^{math.log2(max(ratio, 1e-300)):.1f}); "
          f"elements cancelling below 1e-3 of sum|WG|: {int((cancel < 1e-3).sum())}")
    assert int((cancel < 1e-3).sum()) > 0  # the workload has heavily cancelling elements
    assert (err <= bound * scale + 1e-30).all(), f"max err / sum|WG| = {ratio:.3e} > {bound:.3e}"
