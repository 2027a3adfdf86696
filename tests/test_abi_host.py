"""CPU checks of the C ABI library and of the host-side drop-in surface.

No kernel runs here: the library is loaded, its exports are compared with the
header, and only calls that return before touching the GPU are made (argument
validation, empty sizes, the host-only launch geometry). The registry checks use
CPU and meta tensors: the structural errors of the reference's
core/sanitize.py:276-436 and registry/msda.py:238-241, NoBackendError for CPU
tensors (this build ships no CPU path), and the fake kernels of the private ops.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from deformops_amd.backends.hip import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "deformops_amd.h"


def header_functions() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"^(?:int|const char\*)\s+(msda_\w+)\(", text, flags=re.M)


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_library_exports_every_declared_function(lib):
    declared = header_functions()
    assert {"msda_forward", "msda_backward", "msda_last_error", "msda_abi_version",
            "msda_launch_geometry"} <= set(declared)
    raw = ctypes.CDLL(str(lib.path))
    for name in declared:
        assert hasattr(raw, name), f"{name} declared in {HEADER.name} but not exported"
    assert set(declared) == set(_lib.EXPORTED_SYMBOLS)


def test_abi_version_matches_header(lib):
    version = int(re.search(r"#define MSDA_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert lib.cdll.msda_abi_version() == version


def test_dtype_codes_match_header():
    text = HEADER.read_text()
    codes = {name: int(v) for name, v in re.findall(r"MSDA_(F32|F16|BF16|F64) = (\d+)", text)}
    assert _lib.DTYPE_CODES[torch.float32] == codes["F32"]
    assert _lib.DTYPE_CODES[torch.float16] == codes["F16"]
    assert _lib.DTYPE_CODES[torch.bfloat16] == codes["BF16"]
    assert _lib.DTYPE_CODES[torch.float64] == codes["F64"]
    flags = dict(re.findall(r"(MSDA_SOFTMAX|MSDA_ACCUMULATE_GRAD_VALUE) = (\d+)", text))
    assert _lib.FLAG_SOFTMAX == int(flags["MSDA_SOFTMAX"])
    assert _lib.FLAG_ACCUMULATE_GRAD_VALUE == int(flags["MSDA_ACCUMULATE_GRAD_VALUE"])


def forward_call(lib, *, vdt=2, idt=0, ldt=2, sizes=(4, 21504, 8, 32, 21504, 3, 4), flags=0, ptr=1):
    p = ctypes.c_void_p(ptr) if ptr else None
    return lib.forward(p, vdt, p, p, idt, p, ldt, p, p, *sizes, flags, None)


def backward_call(lib, *, vdt=2, idt=0, ldt=2, sizes=(4, 21504, 8, 32, 21504, 3, 4), flags=0, ptr=1):
    p = ctypes.c_void_p(ptr) if ptr else None
    return lib.backward(p, vdt, p, p, idt, p, ldt, p, p, p, p, p, *sizes, flags, None)


@pytest.mark.parametrize(
    ("kwargs", "fragment"),
    [
        ({"vdt": 9}, "dtype"),
        ({"idt": 5}, "index"),
        ({"ldt": 7}, "dtype"),
        ({"sizes": (4, 21504, 8, 32, -1, 3, 4)}, "negative"),
        ({"sizes": (-2, 21504, 8, 32, 21504, 3, 4)}, "negative"),
        ({"flags": 64}, "flag"),
    ],
)
@pytest.mark.parametrize("direction", ["forward", "backward"])
def test_invalid_calls_fail_before_any_launch(lib, direction, kwargs, fragment):
    call = forward_call if direction == "forward" else backward_call
    rc = call(lib, **kwargs)
    assert rc == 1  # MSDA_ERR_INVALID
    message = lib.cdll.msda_last_error().decode()
    assert fragment in message.lower(), message
    with pytest.raises(RuntimeError, match="msda"):
        lib.check(rc)


def workspace_call(lib, *, vdt=2, sizes=(4, 21504, 8, 32, 21504, 3, 4), flags=0, ws_bytes=0, ptr=1):
    p = ctypes.c_void_p(ptr) if ptr else None
    return lib.backward_workspace(p, vdt, p, p, 0, p, 2, p, p, p, p, p, *sizes, flags, p, ws_bytes, None)


@pytest.mark.parametrize("softmax", [False, True], ids=["linear", "softmax"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("sizes", [(4, 21504, 8, 32, 21504, 3, 4), (4, 17821, 8, 32, 300, 4, 4),
                                   (1, 100, 3, 5, 7, 2, 3), (2, 10, 1, 4, 0, 1, 1)])
def test_workspace_size_holds_the_indices_and_the_counters(lib, dtype, sizes, softmax):
    """One uint32 index per sample, then a counters region at least as large as the
    weight gradient (the capacity the plain call has) and as the bucket and queue
    counters of the largest tile count the host cannot rule out: L (S / 8 + 1) tiles of
    8 x 8 (a one-row level), or the 4 x 4 tiles of small levels, 4 counters each, plus
    288 queue ints, per (b, h); with softmax, then one statistic (float, double for
    float64) per (b, q, h)."""
    from deformops_amd.backends.hip import _bridge  # noqa: PLC0415

    B, S, H, D, Q, L, P = sizes  # noqa: N806
    samples = B * Q * H * L * P
    flags = _lib.FLAG_SOFTMAX if softmax else 0
    size = lib.workspace_size(dtype, *sizes, flags)
    assert size == _bridge._workspace_bytes(dtype, B, S, H, Q, L, P, softmax)  # noqa: SLF001
    assert size % 256 == 0
    align = lambda v: (v + 255) // 256 * 256  # noqa: E731
    tiles = L * max(S // 8 + 1, 4 * (384 // max(1, B * H) + 1))
    counters = B * H * (4 * tiles + 9 * 32) * 4
    stats = align(B * Q * H * (8 if dtype == torch.float64 else 4)) if softmax else 0
    assert size == align(samples * 4) + align(max(samples * dtype.itemsize, counters)) + stats
    if sizes == (4, 21504, 8, 32, 21504, 3, 4) and dtype == torch.bfloat16 and not softmax:
        assert size == 49_545_216  # the size the header quotes


def test_workspace_calls_validate_like_the_plain_backward(lib):
    assert workspace_call(lib, ws_bytes=-1) == 1
    assert "workspace" in lib.cdll.msda_last_error().decode()
    assert workspace_call(lib, vdt=9) == 1
    assert "dtype" in lib.cdll.msda_last_error().decode()
    assert workspace_call(lib, flags=64) == 1
    assert workspace_call(lib, sizes=(0, 21504, 8, 32, 21504, 3, 4)) == 0
    out = ctypes.c_int64(7)
    assert lib.cdll.msda_backward_workspace_size(9, 1, 1, 1, 1, 1, 1, 1, 0, ctypes.byref(out)) == 1
    assert lib.cdll.msda_backward_workspace_size(2, 1, 1, -1, 1, 1, 1, 1, 0, ctypes.byref(out)) == 1
    assert lib.cdll.msda_backward_workspace_size(2, 1, 1, 1, 1, 1, 1, 1, 0, None) == 1


def test_empty_calls_return_ok_without_a_device(lib):
    assert forward_call(lib, sizes=(0, 21504, 8, 32, 21504, 3, 4)) == 0
    assert forward_call(lib, sizes=(4, 21504, 8, 32, 0, 3, 4)) == 0
    assert lib.cdll.msda_last_error().decode() == ""


def geometry(lib, dtype, sizes, backward):
    cpl, lpu, wpb = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    nb = ctypes.c_int64()
    rc = lib.cdll.msda_launch_geometry(dtype, *sizes, int(backward), ctypes.byref(cpl), ctypes.byref(lpu),
                                       ctypes.byref(wpb), ctypes.byref(nb))
    return rc, cpl.value, lpu.value, wpb.value, nb.value


@pytest.mark.parametrize("dtype", [0, 1, 2, 3], ids=["f32", "f16", "bf16", "f64"])
def test_launch_geometry_of_the_headline_shape(lib, dtype):
    sizes = (4, 21504, 8, 32, 21504, 3, 4)
    rc, cpl, lpu, wpb, nb = geometry(lib, dtype, sizes, backward=False)
    assert rc == 0
    assert 32 % cpl == 0 and cpl * lpu >= 1 and 1 <= wpb <= 16 and nb > 0
    rc, cpl, npos, wpb, nb = geometry(lib, dtype, sizes, backward=True)
    assert rc == 0
    assert 32 % cpl == 0 and npos > 0 and 1 <= wpb <= 16 and nb > 0


def test_launch_geometry_rejects_what_the_kernels_do_not_cover(lib):
    # 1030 channels per head: an odd count needs one lane per channel, more than a wave.
    rc, *_ = geometry(lib, 2, (1, 64, 1, 1030, 16, 1, 4), backward=False)
    assert rc == 2  # MSDA_ERR_UNSUPPORTED
    assert "channels" in lib.cdll.msda_last_error().decode().lower()
    rc, *_ = geometry(lib, 2, (1, 64, 1, 1030, 16, 1, 4), backward=True)
    assert rc == 2
    rc, *_ = geometry(lib, 0, (1, 64, 1, 32, 16, 1, 65), backward=True)  # many points: supported
    assert rc == 0
    rc, *_ = geometry(lib, 11, (1, 64, 1, 8, 16, 1, 4), backward=False)
    assert rc == 1


def test_launch_geometry_widens_units_whose_samples_overflow_a_wave(lib):
    # bf16, D = 8: one lane would serve a unit, so a wave would stage 64 units x 40
    # samples (77 KB with their locations and weights). The plan gives each unit more
    # lanes until one wave fits; the backward's grad_sample plan does the same.
    for backward in (False, True):
        rc, cpl, lpu, wpb, nb = geometry(lib, 2, (1, 4, 1, 8, 1, 5, 8), backward=backward)
        assert rc == 0, lib.cdll.msda_last_error()
        if not backward:
            assert cpl == 8 and lpu >= 2
    # Even one unit per wave cannot stage 2048 float32 samples: unsupported, and the
    # registry's predicate says so before any launch.
    rc, *_ = geometry(lib, 0, (1, 64, 1, 32, 16, 1, 2048), backward=True)
    assert rc == 2
    assert "lds" in lib.cdll.msda_last_error().decode().lower()


@pytest.mark.parametrize(
    ("levels", "points", "dtype", "head_dim", "expected"),
    [
        (4, 7, torch.bfloat16, 8, True),
        (5, 8, torch.float32, 8, True),
        (1, 1024, torch.float32, 32, True),
        (1, 2048, torch.float32, 32, False),
        (1, 1024, torch.float64, 16, False),
    ],
)
def test_backend_predicate_matches_the_lds_budget(levels, points, dtype, head_dim, expected):
    from deformops_amd.backends.hip._bridge import supports_context  # noqa: PLC0415
    from deformops_amd.registry import MSDAContext  # noqa: PLC0415

    if torch.version.hip is None:
        pytest.skip("the predicate is for ROCm builds of torch")
    context = MSDAContext(device=torch.device("cuda"), num_levels=levels, num_heads=1, num_points=points,
                          dtype=dtype, sm_version=(9, 5), is_training=True, num_queries=1, head_dim=head_dim)
    assert supports_context(context) is expected


@pytest.mark.parametrize("dtype", [0, 2], ids=["f32", "bf16"])
def test_image_size_limit_is_the_references_element_count(lib, dtype):
    """An image of S H D = 2^31 - 2 elements (2^31 - 1 is prime) is accepted (the
    reference's limit is 2^31 - 1 elements whatever the dtype,
    backends/cuda/include/msda_launch.cuh:85-89), 2^31 are not; the registry's
    predicate agrees, so such a call is NoBackendError."""
    from deformops_amd.backends.hip._bridge import supports_context  # noqa: PLC0415
    from deformops_amd.registry import MSDAContext  # noqa: PLC0415

    for backward in (False, True):
        assert geometry(lib, dtype, (1, 2**30 - 1, 2, 1, 16, 1, 4), backward)[0] == 0, lib.last_error()
        assert geometry(lib, dtype, (1, 2**28, 8, 1, 16, 1, 4), backward)[0] == 2  # 2^31 elements
        assert "2^31 - 1 elements" in lib.last_error()
    if torch.version.hip is None:
        pytest.skip("the predicate is for ROCm builds of torch")
    torch_dtype = torch.float32 if dtype == 0 else torch.bfloat16

    def context(positions: int, heads: int, head_dim: int) -> MSDAContext:
        return MSDAContext(device=torch.device("cuda"), num_levels=1, num_heads=heads, num_points=4,
                           dtype=torch_dtype, sm_version=(9, 5), is_training=True, num_queries=16,
                           head_dim=head_dim, num_positions=positions)

    assert supports_context(context(2**30 - 1, 2, 1))
    assert not supports_context(context(2**23, 8, 32))


def test_missing_library_raises_kernel_error(monkeypatch, tmp_path):
    from deformops_amd.core.errors import KernelNotProvidedError  # noqa: PLC0415

    monkeypatch.setenv("DEFORMOPS_AMD_LIBRARY", str(tmp_path / "absent.so"))
    monkeypatch.delenv("DEFORMOPS_COMPILE", raising=False)
    monkeypatch.setattr(_lib, "_loaded", None)
    with pytest.raises(KernelNotProvidedError):
        _lib.load()


# Host side of the drop-in surface.


def small_operands(device="cpu", dtype=torch.float32):
    shapes = torch.tensor([[4, 4], [2, 2]], device=device)
    starts = torch.tensor([0, 16], device=device)
    value = torch.randn(1, 20, 2, 8, device=device, dtype=dtype)
    loc = torch.rand(1, 3, 2, 2, 4, 2, device=device, dtype=dtype)
    attn = torch.rand(1, 3, 2, 8, device=device, dtype=dtype)
    return value, shapes, starts, loc, attn


def test_cpu_tensors_run_the_eager_backend():
    from deformops_amd.backends.eager.msda import forward  # noqa: PLC0415
    from deformops_amd.registry import msda  # noqa: PLC0415

    ops = small_operands()
    torch.testing.assert_close(msda(*ops), forward(*ops), rtol=0, atol=0)


@pytest.mark.parametrize(
    ("mutate", "operand"),
    [
        (lambda v, sh, st, lc, a: (v[0], sh, st, lc, a), "value"),
        (lambda v, sh, st, lc, a: (v, sh.float(), st, lc, a), "spatial_shapes"),
        (lambda v, sh, st, lc, a: (v, sh, st[:1], lc, a), "level_start_index"),
        (lambda v, sh, st, lc, a: (v, sh, st, lc[..., :1], a), "sampling_locations"),
        (lambda v, sh, st, lc, a: (v, sh, st, lc, a[..., :5]), "attention_weights"),
        (lambda v, sh, st, lc, a: (v, sh, st, lc, a.double()), "attention_weights"),
    ],
)
def test_malformed_operands_raise_value_error_naming_the_operand(mutate, operand):
    from deformops_amd.registry import msda  # noqa: PLC0415

    with pytest.raises(ValueError, match=operand):
        msda(*mutate(*small_operands()))


def test_keyword_errors_are_type_errors():
    from deformops_amd.registry import msda  # noqa: PLC0415

    with pytest.raises(TypeError):
        msda(*small_operands(), not_an_option=1)
    with pytest.raises(TypeError):
        msda(*small_operands(), backend="hip")


def test_private_ops_have_fake_kernels():
    import deformops_amd  # noqa: F401, PLC0415

    value, shapes, starts, loc, attn = (t.to("meta") for t in small_operands())
    ops = torch.ops.deformops_hip
    out = ops.msda_forward(value, shapes, starts, loc, attn, 128, 4, 8, 256)
    assert out.shape == (1, 3, 16) and out.device.type == "meta" and out.dtype == value.dtype
    grads = ops.msda_backward(value, shapes, starts, loc, attn, out, 128, 4, 8, 256)
    assert [g.shape for g in grads] == [value.shape, loc.shape, attn.shape]
    out = ops.msda_softmax_forward(value, shapes, starts, loc, attn, 128, 4, 8, 256)
    assert out.shape == (1, 3, 16)


def test_public_ops_carry_the_reference_schema():
    import deformops_amd  # noqa: F401, PLC0415

    for name in ("msda", "msda_softmax"):
        schema = str(getattr(torch.ops.deformops, name).default._schema)
        assert schema == (
            f"deformops::{name}(Tensor value, Tensor spatial_shapes, Tensor level_start_index, "
            "Tensor sampling_locations, Tensor attention_weights) -> Tensor"
        )


def test_probe_library_exports_its_header():
    """bench_probe/libmsda_probe.so (bench.py's row-gather probe, outside the product
    package) exports what bench_probe/msda_probe.h declares."""
    probe_dir = Path(__file__).resolve().parents[1] / "bench_probe"
    declared = re.findall(r"^int\s+(msda_\w+)\(", (probe_dir / "msda_probe.h").read_text(), flags=re.M)
    assert declared == ["msda_probe_row_gather"]
    probe = ctypes.CDLL(str(probe_dir / "libmsda_probe.so"))
    for name in declared:
        assert hasattr(probe, name)

