"""Screen-space gradient statistics used for densification.

``accumulate_grad2d_stats`` performs the running-state update of
gsplat/strategy/default.py:218-268 (``DefaultStrategy._update_state``):
the per-row 2D mean gradient (``absgrad`` or ``grad``) is scaled to the
[-1, 1] screen range, and its norm plus a visit count are added to per-
Gaussian accumulators.
"""

from __future__ import annotations

from typing import Dict, Optional

import torch
from torch import Tensor


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
    grads = grads.clone()
    grads[..., 0] *= info["width"] / 2.0 * info["n_cameras"]
    grads[..., 1] *= info["height"] / 2.0 * info["n_cameras"]
    if grad2d is None:
        grad2d = torch.zeros(n_gaussians, device=grads.device)
    if count is None:
        count = torch.zeros(n_gaussians, device=grads.device)
    if packed:
        gs_ids = info["gaussian_ids"]
    else:
        sel = (info["radii"] > 0.0).all(dim=-1)
        gs_ids = torch.where(sel)[-1]
        grads = grads[sel]
    grad2d.index_add_(0, gs_ids, grads.norm(dim=-1))
    count.index_add_(0, gs_ids, torch.ones_like(gs_ids, dtype=torch.float32))
    return grad2d, count
