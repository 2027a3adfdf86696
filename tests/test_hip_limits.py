"""The largest image the kernels address, through ``registry.msda``.

The kernels index the rows of one batch image of ``value`` (and of
``grad_value``) with 32-bit row offsets (position * H + head) and form 64-bit byte
addresses from them, so an image may hold up to 2^31 - 1 elements, the reference's
limit (backends/cuda/include/msda_launch.cuh:85-89); the host rejects larger ones
(tests/test_abi_host.py). Here one level of 2048 x 4095 positions with H = 8 and
D = 32 makes an image 2^31 - 524,288 elements: 4.3 GB in bf16 and 8.6 GB in float32,
past 2^31 bytes either way, and a batch of two puts the second image past 2^32
bytes. Half the queries sample the first rows of the level and half its last rows
and columns, where the offsets are largest.

Each group's corners all lie in an 8-row band of the level (or outside the level,
which the band reproduces: a row beyond the band is beyond the level too). So the
float64 oracle runs on that band alone, with the band's own level shape: its
results are those of the full problem, except that the location gradient's y
component scales with the level height (2048 against 8). grad_value must equal the
band's gradient inside each band and be exactly zero everywhere else.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from deformops_amd.registry import msda
from tests.test_hip_msda import BWD_TOL, FWD_TOL, rel_err

pytestmark = pytest.mark.gpu

BAND = 8


def _pixels(g: torch.Generator, n: int, lo: float, hi: float) -> torch.Tensor:
    return lo + (hi - lo) * torch.rand(n, generator=g, dtype=torch.float64)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_largest_image_addressable_with_32_bit_row_offsets(device, dtype):
    Hh, W = 2048, 4095
    B, H, D, P = 2, 8, 32, 4
    S = Hh * W
    es = torch.empty((), dtype=dtype).element_size()
    assert 0 < 2**31 - S * H * D <= 2**20 and S * H * D * es > 2**31
    Qg = 32  # queries per band
    g = torch.Generator().manual_seed(2047)
    # Pixel coordinates x = loc_x * W - 0.5 (and y alike). Top band rows 0..7: y in
    # [-1, 5], so corner rows stay in -1..6. Bottom band rows Hh-8..Hh-1: y in
    # [Hh-6, Hh), so corner rows reach Hh (outside the level) at most.
    bands = {0: (-1.0, 5.0, -1.0, float(W)), Hh - BAND: (Hh - 6.0, Hh - 1e-3, W - 9.0, W - 1e-3)}
    locs = []
    for y_lo, y_hi, x_lo, x_hi in bands.values():
        n = B * Qg * H * P
        x = _pixels(g, n, x_lo, x_hi)
        y = _pixels(g, n, y_lo, y_hi)
        xy = torch.stack([(x + 0.5) / W, (y + 0.5) / Hh], -1).reshape(B, Qg, H, 1, P, 2)
        locs.append(xy)
    loc = torch.cat(locs, 1).to(torch.float32)  # (B, 2 Qg, H, 1, P, 2)
    attn = torch.softmax(torch.randn(B, 2 * Qg, H, P, generator=g, dtype=torch.float64), -1).to(dtype)
    grad_out = torch.randn(B, 2 * Qg, H * D, generator=g, dtype=torch.float64).to(dtype)
    value = torch.randn(B, S, H, D, device=device, dtype=dtype)  # drawn on the GPU: up to 17 GB
    shapes = torch.tensor([[Hh, W]], device=device)
    starts = torch.tensor([0], device=device)

    leaves = [value.requires_grad_(True), loc.to(device).requires_grad_(True), attn.to(device).requires_grad_(True)]
    out = msda(leaves[0], shapes, starts, leaves[1], leaves[2])
    out.backward(grad_out.to(device))
    torch.cuda.synchronize()
    gv = leaves[0].grad.view(B, Hh, W, H, D)
    gl, ga = leaves[1].grad.cpu(), leaves[2].grad.cpu()

    # The pixel rows the kernel computed (float32, as the oracle's pixel map does).
    y_pix = loc[..., 1] * torch.tensor(Hh, dtype=torch.float32) - 0.5
    for i, r0 in enumerate(bands):
        qs = slice(i * Qg, (i + 1) * Qg)
        band_value = value.detach().view(B, Hh, W, H, D)[:, r0:r0 + BAND].reshape(B, BAND * W, H, D).cpu()
        band_loc = loc[:, qs].clone().to(torch.float64)
        band_loc[..., 1] = ((y_pix[:, qs].to(torch.float64) - r0) + 0.5) / BAND
        band_shapes, band_starts = torch.tensor([[BAND, W]]), torch.tensor([0])
        ref = oracle.forward(band_value, band_shapes, band_starts, band_loc, attn[:, qs])
        rgv, rgl, rga = oracle.backward(band_value, band_shapes, band_starts, band_loc, attn[:, qs], grad_out[:, qs])
        assert rel_err(out[:, qs], ref) <= FWD_TOL[dtype]
        assert rel_err(gv[:, r0:r0 + BAND].reshape(B, BAND * W, H, D), rgv) <= BWD_TOL[dtype]
        # d/d(loc_y) carries the level height: Hh in the full problem, BAND in the band.
        rgl = rgl.clone()
        rgl[..., 1] *= Hh / BAND
        assert rel_err(gl[:, qs], rgl) <= BWD_TOL[dtype]
        assert rel_err(ga[:, qs], rga.reshape(ga[:, qs].shape)) <= BWD_TOL[dtype]
    # No sample reaches the rows between the bands.
    assert gv[:, BAND:Hh - BAND].abs().amax().item() == 0.0


# Many samples per (query, head): the staged records of one unit grow with L * P, and
# where a wave's units would not fit its LDS budget a unit takes more lanes than its
# channels need (msda_launch_geometry; tests/test_abi_host.py). L * P = 128 gives a
# bf16 unit of D = 32 8 lanes for the 4 its channels need; L * P = 512 with D = 8
# takes 32 lanes for 2.
MANY = [
    pytest.param(((12, 12), (6, 6), (3, 3), (2, 2)), 32, 32, torch.bfloat16, id="lp128-bf16"),
    pytest.param(((12, 12), (6, 6), (3, 3), (2, 2)), 32, 32, torch.float32, id="lp128-f32"),
    pytest.param(((16, 16), (4, 4)), 256, 8, torch.float32, id="lp512-d8-f32"),
]


@pytest.mark.parametrize(("levels", "P", "D", "dtype"), MANY)
def test_many_samples_per_unit(device, levels, P, D, dtype):
    from tests.test_hip_msda import check_against_oracle  # noqa: PLC0415
    from tests.workloads import make_workload  # noqa: PLC0415

    w = make_workload(0, levels=levels, batch=2, queries=37, heads=3, channels=D, points=P,
                      locations="uniform", seed=P).to(device, dtype)
    for softmax in (False, True):
        check_against_oracle(*w.operands(softmax=softmax), w.grad_output, softmax=softmax, dtype=dtype,
                             label=f"L*P={len(levels) * P} D={D}")
