"""Level tables whose levels share positions of S, at real fan-in.

The reference's validator calls such tables malformed (core/sanitize.py:395-436),
but its eager and atomic paths sum every level's contribution into a shared
element (backends/eager/msda_pytorch.py:83-112). On the matrix-core owners the
bucket sort takes overlapping levels as it takes any (each level's tiles are its own
buckets); the count pass zeroes grad_value and every level's owner adds its fp32 sum
with one atomic per element (16-bit: per channel pair), so a shared element carries
at most two roundings per level instead of one per contribution, as a 16-bit atomic
scatter would. These tests run config 2's pyramid and fan-in (B = 2, 5,376 queries,
8 heads, bf16 and f16) against the float64 oracle.
"""

from __future__ import annotations

import dataclasses

import pytest
import torch

from tests.test_hip_msda import BF16, F16, F32, abi_backward, check_against_oracle, rel_err
from tests.workloads import make_workload

pytestmark = pytest.mark.gpu

OVERLAPS_AT_SCALE = [
    # the 32 x 32 level listed twice, at the same start
    pytest.param(((64, 64), (32, 32), (32, 32)), (0, 4096, 4096), 5120, id="duplicated-level"),
    # the 16 x 16 level starting 100 positions inside the 32 x 32 one
    pytest.param(((64, 64), (32, 32), (16, 16)), (0, 4096, 4996), 5252, id="level-inside-another"),
]


def overlapping(levels, starts, S, dtype, device, **sizes):
    w = make_workload(2, levels=levels, **sizes)
    B, _, H, D = w.value.shape
    value = torch.randn(B, S, H, D, generator=torch.Generator().manual_seed(11), dtype=torch.float64)
    return dataclasses.replace(w, value=value, level_start_index=torch.tensor(starts)).to(device, dtype)


def bound(dtype):
    """Two roundings to the dtype per level, three levels."""
    return 6 * (2.0**-8 if dtype == BF16 else 2.0**-10)


@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "f16"])
@pytest.mark.parametrize(("levels", "starts", "S"), OVERLAPS_AT_SCALE)
def test_overlapping_levels_at_scale_keep_fp32_sums(device, levels, starts, S, dtype):
    w = overlapping(levels, starts, S, dtype, device)
    for softmax in (False, True):
        errs = check_against_oracle(*w.operands(softmax=softmax), w.grad_output, softmax=softmax, dtype=dtype,
                                    label=f"overlap {levels} {starts}")
        print(f"{levels} {starts} {dtype} softmax={softmax}: {errs}")
        assert errs["grad_value"] <= bound(dtype), errs


@pytest.mark.parametrize("dtype", [BF16, F32], ids=["bf16", "f32"])
def test_overlapping_levels_accumulate_into_grad_value(device, dtype):
    """MSDA_ACCUMULATE_GRAD_VALUE with overlapping levels: the owners add onto the
    previous contents (no zeroing)."""
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    levels, starts, S = ((64, 64), (32, 32), (16, 16)), (0, 4096, 4996), 5252
    w = overlapping(levels, starts, S, dtype, device, batch=1, queries=2000)
    plain = abi_backward(w, 0)
    previous = torch.randn(w.value.shape, generator=torch.Generator().manual_seed(3)).to(device, dtype)
    added = abi_backward(w, _lib.FLAG_ACCUMULATE_GRAD_VALUE, grad_value=previous.clone())
    expected = previous.double().cpu() + plain[0].double().cpu()
    assert rel_err(added[0], expected) <= (bound(dtype) if dtype == BF16 else 1e-5)
    torch.testing.assert_close(added[1], plain[1], rtol=0, atol=0)
    torch.testing.assert_close(added[2], plain[2], rtol=0, atol=0)


@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "f16"])
def test_overlapping_levels_with_the_atomic_counting_sort(device, dtype):
    """The same table through the sort's atomic counting mode (msda_set_path_override)."""
    from deformops_amd.backends.hip import _lib  # noqa: PLC0415

    levels, starts, S = OVERLAPS_AT_SCALE[0].values
    w = overlapping(levels, starts, S, dtype, device, batch=1)
    with _lib.path_override(_lib.PATH_ATOMIC_SORT):
        errs = check_against_oracle(*w.operands(), w.grad_output, softmax=False, dtype=dtype, label="atomic sort")
    assert errs["grad_value"] <= bound(dtype), errs
