"""Screen-space gradient statistics used for densification.

``accumulate_grad2d_stats`` performs the running-state update of
gsplat/strategy/default.py:218-268 (``DefaultStrategy._update_state``):
the per-row 2D mean gradient (``absgrad`` or ``grad``) is scaled to the
[-1, 1] screen range, and its norm plus a visit count are added to per-
Gaussian accumulators.  One HIP launch (``gsplat_grad2d_stats``) reads the
row gradients once, where the reference runs a clone, two column scales, a
norm and two ``index_add_``.
"""

from __future__ import annotations

from typing import Dict, Optional

import torch
from torch import Tensor

from ..cuda import _ops


@torch.no_grad()
def accumulate_grad2d_stats(
    info: Dict,
    grad2d: Optional[Tensor],
    count: Optional[Tensor],
    n_gaussians: int,
    packed: bool,
    absgrad: bool = True,
):
    """Adds ||dL/dmean2d * (W/2 * C, H/2 * C)|| to ``grad2d[g]`` and 1 to
    ``count[g]`` for every visible (camera, Gaussian) row.

    Returns the (possibly freshly allocated) ``(grad2d, count)``.
    """
    means2d = info["means2d"]
    grads = means2d.absgrad if absgrad else means2d.grad
    if grad2d is None:
        grad2d = torch.zeros(n_gaussians, device=grads.device)
    if count is None:
        count = torch.zeros(n_gaussians, device=grads.device)
    sx = info["width"] / 2.0 * info["n_cameras"]
    sy = info["height"] / 2.0 * info["n_cameras"]
    if packed:
        _ops.grad2d_stats(grads.contiguous(), info["gaussian_ids"].contiguous(), None,
                          n_gaussians, sx, sy, grad2d, count)
    else:
        _ops.grad2d_stats(grads.contiguous(), None, info["radii"].contiguous(),
                          n_gaussians, sx, sy, grad2d, count)
    return grad2d, count


def fuse_grad2d_stats(
    info: Dict,
    grad2d: Optional[Tensor],
    count: Optional[Tensor],
    n_gaussians: int,
    absgrad: bool = True,
):
    """Requests the same statistics update as ``accumulate_grad2d_stats``,
    performed inside the backward pass by the packed projection's own
    gradient kernel instead of a separate pass over the rows afterwards.

    Call it between ``rasterization()`` and ``backward()``.  Available for the
    packed path with one batch (``info["grad2d_stats_slot"]`` present);
    returns ``(grad2d, count, fused)``, and when ``fused`` is False the
    caller runs ``accumulate_grad2d_stats`` after the backward as usual."""
    slot = info.get("grad2d_stats_slot")
    means2d = info["means2d"]
    if grad2d is None:
        grad2d = torch.zeros(n_gaussians, device=means2d.device)
    if count is None:
        count = torch.zeros(n_gaussians, device=means2d.device)
    if slot is None or grad2d.numel() != n_gaussians or count.numel() != n_gaussians:
        return grad2d, count, False
    slot.request = (grad2d, count, absgrad)
    return grad2d, count, True
