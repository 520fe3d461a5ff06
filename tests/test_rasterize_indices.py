"""rasterize_to_indices_3dgs (RasterizeToIndices3DGS.cu:36-196) through the
C-ABI against the host restatement (oracle/exact.py): the (Gaussian, pixel)
pairs, in pixel-major, front-to-back order, for the full range from full
transmittance, for batch sub-ranges from arbitrary transmittances, for
several images, and for the empty cases."""

import numpy as np
import pytest
import torch

from oracle import exact
from tests._util import DEV, projected_2d

pytestmark = pytest.mark.gpu


def _run(d, range_start, range_end, T):
    from gsplat_amd.cuda._wrapper import rasterize_to_indices_in_range
    C, N = d["C"], d["means2d"].shape[-2]
    m2 = d["means2d"].reshape(C, -1, 2)
    con = d["conics"].reshape(C, -1, 3)
    op = d["opacities"].reshape(C, -1)
    g, p, im = rasterize_to_indices_in_range(
        range_start, range_end, T.to(DEV), m2.to(DEV), con.to(DEV), op.to(DEV),
        d["W"], d["H"], d["tile"], d["offsets"].to(DEV), d["flatten_ids"].to(DEV))
    eg, ep = exact.rasterize_to_indices(
        range_start, range_end, T.numpy(), m2.numpy(), con.numpy(), op.numpy(),
        d["W"], d["H"], d["tile"], d["offsets"].numpy(), d["flatten_ids"].numpy(),
        m2.shape[1])
    HW = d["H"] * d["W"]
    np.testing.assert_array_equal(g.cpu().numpy(), eg)
    np.testing.assert_array_equal(p.cpu().numpy(), ep % HW)
    np.testing.assert_array_equal(im.cpu().numpy(), ep // HW)
    return eg


@pytest.mark.parametrize("tile", [16, 8, 4])
def test_indices_full_range(tile):
    d = projected_2d(seed=3, N=600, C=1, W=64, H=48, tile=tile)
    eg = _run(d, 0, 10 ** 10, torch.ones(1, d["H"], d["W"]))
    assert eg.size > 1000


@pytest.mark.parametrize("tile", [16, 8, 4])
def test_indices_ragged_image(tile):
    # image edges inside the last tile row and column: those tiles' outside
    # pixels composite nothing and own empty ranges
    d = projected_2d(seed=7, N=400, C=2, W=37, H=29, tile=tile)
    eg = _run(d, 0, 10 ** 10, torch.ones(2, d["H"], d["W"]))
    assert eg.size > 500


def test_indices_batch_ranges_and_transmittances():
    d = projected_2d(seed=4, N=500, C=2, W=32, H=32)
    g = torch.Generator().manual_seed(2)
    T = torch.rand(2, d["H"], d["W"], generator=g) * 0.9 + 0.1
    T[0, :4, :4] = 1e-4  # already at the cutoff
    for lo, hi in [(0, 1), (1, 2), (1, 10 ** 10), (0, 10 ** 10)]:
        _run(d, lo, hi, T)


def test_indices_empty():
    from gsplat_amd.cuda import _ops
    d = projected_2d(seed=6, N=50, C=1, W=32, H=32)
    g, p = _ops.rasterize_to_indices_3dgs(
        50, 60, torch.ones(1, 32, 32, device=DEV), d["means2d"][None].to(DEV),
        d["conics"][None].to(DEV), d["opacities"][None].to(DEV), 32, 32, 16,
        d["offsets"].to(DEV), d["flatten_ids"].to(DEV))
    assert g.numel() == 0 and p.numel() == 0
