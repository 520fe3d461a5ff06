"""Host side of every gsplat op: output allocation + one C-ABI call.

Each function here has the argument list and return convention of the
reference op of the same name (schemas in gsplat/cuda/ext.cpp:711-754,
host wrappers in gsplat/cuda/csrc/{Projection,Intersect,Rasterization,
SphericalHarmonics,Adam}.cpp).  Outputs are allocated through the torch
caching allocator on the inputs' device; the kernels run on the current
stream of that device.  Optional outputs that the reference returns as an
undefined tensor are returned as ``None``.

These functions are what ``torch.ops.gsplat.*`` dispatches to for the CUDA
(HIP) key (see ``_backend.py``); the autograd wrappers call them directly to
skip the dispatcher round trip.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
from torch import Tensor

from .._lib import AdamTensor, call, check_input, ptr, query

_F32 = torch.float32
_I32 = torch.int32
_I64 = torch.int64


def _stream(t: Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _prod(shape) -> int:
    return int(math.prod(shape))


# --------------------------------------------------------------------------
# Spherical harmonics  (SphericalHarmonics.cpp:33-91)
# --------------------------------------------------------------------------
def spherical_harmonics_fwd(
    degrees_to_use: int, dirs: Tensor, coeffs: Tensor, masks: Optional[Tensor]
) -> Tensor:
    check_input(dirs, "dirs", _F32)
    check_input(coeffs, "coeffs", _F32)
    check_input(masks, "masks", torch.bool)
    M = dirs.numel() // 3
    K = coeffs.shape[-2]
    colors = torch.empty_like(dirs)
    call("gsplat_sh_fwd", M, K, degrees_to_use, ptr(dirs), ptr(coeffs),
         ptr(masks), ptr(colors), _stream(dirs))
    return colors


def spherical_harmonics_bwd(
    degrees_to_use: int,
    dirs: Tensor,
    coeffs: Tensor,
    masks: Optional[Tensor],
    v_colors: Tensor,
    compute_v_dirs: bool,
) -> Tuple[Tensor, Optional[Tensor]]:
    check_input(dirs, "dirs", _F32)
    check_input(coeffs, "coeffs", _F32)
    check_input(masks, "masks", torch.bool)
    check_input(v_colors, "v_colors", _F32)
    M = dirs.numel() // 3
    K = coeffs.shape[-2]
    v_coeffs = torch.empty_like(coeffs)
    v_dirs = torch.empty_like(dirs) if compute_v_dirs else None
    call("gsplat_sh_bwd", M, K, degrees_to_use, ptr(dirs), ptr(coeffs),
         ptr(masks), ptr(v_colors), ptr(v_coeffs), ptr(v_dirs), _stream(dirs))
    return v_coeffs, v_dirs


# --------------------------------------------------------------------------
# Projection  (Projection.cpp:129-576)
# --------------------------------------------------------------------------
def _proj_dims(means: Tensor, viewmats: Tensor):
    batch_dims = tuple(means.shape[:-2])
    N = means.shape[-2]
    C = viewmats.shape[-3]
    B = _prod(batch_dims)
    return batch_dims, B, C, N


def _check_proj_inputs(means, covars, quats, scales, opacities, viewmats, Ks):
    check_input(means, "means", _F32)
    if covars is not None:
        check_input(covars, "covars", _F32)
    else:
        if quats is None or scales is None:
            raise RuntimeError("projection: covars or (quats, scales) required")
        check_input(quats, "quats", _F32)
        check_input(scales, "scales", _F32)
    check_input(opacities, "opacities", _F32)
    check_input(viewmats, "viewmats", _F32)
    check_input(Ks, "Ks", _F32)


def projection_ewa_simple_fwd(means: Tensor, covars: Tensor, Ks: Tensor, width: int,
                              height: int, camera_model: int) -> Tuple[Tensor, Tensor]:
    """means [..., C, N, 3], covars [..., C, N, 3, 3], Ks [..., C, 3, 3] ->
    means2d [..., C, N, 2], covars2d [..., C, N, 2, 2] (Projection.cpp:41-80)."""
    check_input(means, "means", _F32)
    check_input(covars, "covars", _F32)
    check_input(Ks, "Ks", _F32)
    C, N = means.shape[-3], means.shape[-2]
    B = _prod(means.shape[:-3])
    lead = tuple(means.shape[:-1])
    means2d = torch.empty(lead + (2,), dtype=_F32, device=means.device)
    covars2d = torch.empty(lead + (2, 2), dtype=_F32, device=means.device)
    call("gsplat_projection_simple_fwd", B, C, N, ptr(means), ptr(covars), ptr(Ks),
         int(width), int(height), int(camera_model), ptr(means2d), ptr(covars2d),
         _stream(means))
    return means2d, covars2d


def projection_ewa_simple_bwd(means: Tensor, covars: Tensor, Ks: Tensor, width: int,
                              height: int, camera_model: int, v_means2d: Tensor,
                              v_covars2d: Tensor) -> Tuple[Tensor, Tensor]:
    """Gradients of ``projection_ewa_simple_fwd`` (Projection.cpp:82-127)."""
    check_input(means, "means", _F32)
    check_input(covars, "covars", _F32)
    check_input(Ks, "Ks", _F32)
    check_input(v_means2d, "v_means2d", _F32)
    check_input(v_covars2d, "v_covars2d", _F32)
    C, N = means.shape[-3], means.shape[-2]
    B = _prod(means.shape[:-3])
    v_means = torch.empty_like(means)
    v_covars = torch.empty_like(covars)
    call("gsplat_projection_simple_bwd", B, C, N, ptr(means), ptr(covars), ptr(Ks),
         int(width), int(height), int(camera_model), ptr(v_means2d), ptr(v_covars2d),
         ptr(v_means), ptr(v_covars), _stream(means))
    return v_means, v_covars


def projection_ewa_3dgs_fused_fwd(
    means: Tensor,
    covars: Optional[Tensor],
    quats: Optional[Tensor],
    scales: Optional[Tensor],
    opacities: Optional[Tensor],
    viewmats: Tensor,
    Ks: Tensor,
    image_width: int,
    image_height: int,
    eps2d: float,
    near_plane: float,
    far_plane: float,
    radius_clip: float,
    calc_compensations: bool,
    camera_model: int,
) -> Tuple[Tensor, Tensor, Tensor, Tensor, Optional[Tensor]]:
    _check_proj_inputs(means, covars, quats, scales, opacities, viewmats, Ks)
    batch_dims, B, C, N = _proj_dims(means, viewmats)
    dev = means.device
    radii = torch.empty(batch_dims + (C, N, 2), dtype=_I32, device=dev)
    means2d = torch.empty(batch_dims + (C, N, 2), dtype=_F32, device=dev)
    depths = torch.empty(batch_dims + (C, N), dtype=_F32, device=dev)
    conics = torch.empty(batch_dims + (C, N, 3), dtype=_F32, device=dev)
    comps = (torch.empty(batch_dims + (C, N), dtype=_F32, device=dev)
             if calc_compensations else None)
    call("gsplat_projection_fused_fwd", B, C, N, ptr(means), ptr(covars),
         ptr(quats), ptr(scales), ptr(opacities), ptr(viewmats), ptr(Ks),
         int(image_width), int(image_height), float(eps2d), float(near_plane),
         float(far_plane), float(radius_clip), int(camera_model),
         ptr(radii), ptr(means2d), ptr(depths), ptr(conics), ptr(comps),
         _stream(means))
    return radii, means2d, depths, conics, comps


def projection_ewa_3dgs_fused_bwd(
    means: Tensor,
    covars: Optional[Tensor],
    quats: Optional[Tensor],
    scales: Optional[Tensor],
    viewmats: Tensor,
    Ks: Tensor,
    image_width: int,
    image_height: int,
    eps2d: float,
    camera_model: int,
    radii: Tensor,
    conics: Tensor,
    compensations: Optional[Tensor],
    v_means2d: Tensor,
    v_depths: Tensor,
    v_conics: Tensor,
    v_compensations: Optional[Tensor],
    viewmats_requires_grad: bool,
):
    _check_proj_inputs(means, covars, quats, scales, None, viewmats, Ks)
    for t, n in ((radii, "radii"), (conics, "conics"), (v_means2d, "v_means2d"),
                 (v_depths, "v_depths"), (v_conics, "v_conics"),
                 (compensations, "compensations"),
                 (v_compensations, "v_compensations")):
        check_input(t, n)
    batch_dims, B, C, N = _proj_dims(means, viewmats)
    v_means = torch.empty_like(means)
    v_covars = v_quats = v_scales = None
    if covars is not None:
        v_covars = torch.empty_like(covars)
    else:
        v_quats = torch.empty_like(quats)
        v_scales = torch.empty_like(scales)
    v_viewmats = torch.zeros_like(viewmats) if viewmats_requires_grad else None
    call("gsplat_projection_fused_bwd", B, C, N, ptr(means), ptr(covars),
         ptr(quats), ptr(scales), ptr(viewmats), ptr(Ks), int(image_width),
         int(image_height), float(eps2d), int(camera_model), ptr(radii),
         ptr(conics), ptr(compensations), ptr(v_means2d), ptr(v_depths),
         ptr(v_conics), ptr(v_compensations), ptr(v_means), ptr(v_covars),
         ptr(v_quats), ptr(v_scales), ptr(v_viewmats), _stream(means))
    return v_means, v_covars, v_quats, v_scales, v_viewmats


def projection_packed_fwd_with_row_map(
    means: Tensor,
    covars: Optional[Tensor],
    quats: Optional[Tensor],
    scales: Optional[Tensor],
    opacities: Optional[Tensor],
    viewmats: Tensor,
    Ks: Tensor,
    image_width: int,
    image_height: int,
    eps2d: float,
    near_plane: float,
    far_plane: float,
    radius_clip: float,
    calc_compensations: bool,
    camera_model: int,
):
    """The packed projection's nine outputs plus ``row_of`` [B*C*N] int32:
    the packed row of every (b, c, g), or -1 (the inverse of the id arrays,
    used by the gathers of the packed rasterization path)."""
    _check_proj_inputs(means, covars, quats, scales, opacities, viewmats, Ks)
    batch_dims, B, C, N = _proj_dims(means, viewmats)
    dev = means.device
    cap = B * C * N
    indptr = torch.empty(B * C + 1, dtype=_I32, device=dev)
    batch_ids = torch.empty(cap, dtype=_I64, device=dev)
    camera_ids = torch.empty(cap, dtype=_I64, device=dev)
    gaussian_ids = torch.empty(cap, dtype=_I64, device=dev)
    radii = torch.empty(cap, 2, dtype=_I32, device=dev)
    means2d = torch.empty(cap, 2, dtype=_F32, device=dev)
    depths = torch.empty(cap, dtype=_F32, device=dev)
    conics = torch.empty(cap, 3, dtype=_F32, device=dev)
    comps = torch.empty(cap, dtype=_F32, device=dev) if calc_compensations else None
    row_of = torch.empty(cap, dtype=_I32, device=dev)
    if cap == 0:
        indptr.zero_()
        nnz = 0
    else:
        ws = torch.empty(query("gsplat_projection_packed_workspace_size", B, C, N),
                         dtype=torch.uint8, device=dev)
        nnz_dev = torch.empty(1, dtype=_I64, device=dev)
        call("gsplat_projection_packed_fwd", B, C, N, ptr(means), ptr(covars),
             ptr(quats), ptr(scales), ptr(opacities), ptr(viewmats), ptr(Ks),
             int(image_width), int(image_height), float(eps2d),
             float(near_plane), float(far_plane), float(radius_clip),
             int(camera_model), ptr(ws), ws.numel(), ptr(indptr),
             ptr(batch_ids), ptr(camera_ids), ptr(gaussian_ids), ptr(radii),
             ptr(means2d), ptr(depths), ptr(conics), ptr(comps), ptr(nnz_dev),
             ptr(row_of), None, _stream(means))
        nnz = int(nnz_dev.item())
    return (
        indptr,
        batch_ids[:nnz],
        camera_ids[:nnz],
        gaussian_ids[:nnz],
        radii[:nnz],
        means2d[:nnz],
        depths[:nnz],
        conics[:nnz],
        comps[:nnz] if comps is not None else None,
        row_of,
    )


def packed_front_fwd(
    means: Tensor,
    covars: Optional[Tensor],
    quats: Optional[Tensor],
    scales: Optional[Tensor],
    opacities: Tensor,
    features: Tensor,
    viewmats: Tensor,
    Ks: Tensor,
    image_width: int,
    image_height: int,
    eps2d: float,
    near_plane: float,
    far_plane: float,
    radius_clip: float,
    calc_compensations: bool,
    camera_model: int,
    sh_degree: Optional[int],
    isect: Optional[dict] = None,
):
    """rasterization()'s packed front end: the packed projection plus every
    row's opacity (opacities[b, g]) and colour, either the clamped SH colour
    of per-Gaussian coefficients ``features`` [..., N, K, 3] (``sh_degree``
    given) or a gather of per-Gaussian features [..., N, D].

    The colour kernel is driven by Gaussian through ``row_of`` and writes
    into capacity-sized rows, so it is queued right behind the projection;
    the visible count travels to a pinned host word in between, and the host
    waits for that copy only, while the colour kernel runs.  Returns the
    outputs of ``projection_packed_fwd_with_row_map`` followed by
    ``row_opacities`` [nnz] and ``row_colors`` [nnz, D].

    With ``isect`` = {"tile_size", "tile_width", "tile_height"} (for row
    opacities that are used as they are, i.e. without compensations), the
    first half of the sorted tile intersection of the rows is queued right
    after the wait, before the host slices the outputs, and its state is
    left in ``isect["state"]`` for ``isect_emit_sorted``.  With SH colours
    of one batch, the rows' tile counts share the colour launch
    (gsplat_sh_rows_fwd_isect_count) and only the row starts follow the
    wait."""
    _check_proj_inputs(means, covars, quats, scales, opacities, viewmats, Ks)
    if opacities is None:
        raise RuntimeError("packed_front_fwd: opacities are required")
    check_input(features, "features", _F32)
    batch_dims, B, C, N = _proj_dims(means, viewmats)
    dev = means.device
    if sh_degree is None:
        D = features.shape[-1]
        if tuple(features.shape) != batch_dims + (N, D):
            raise RuntimeError(f"packed_front_fwd: features {tuple(features.shape)} "
                               f"must be [..., N, D]")
    else:
        D = 3
        K = features.shape[-2]
        if (tuple(features.shape) != batch_dims + (N, K, 3)
                or (int(sh_degree) + 1) ** 2 > K):
            raise RuntimeError(f"packed_front_fwd: coefficients {tuple(features.shape)} "
                               f"do not hold degree {sh_degree}")
    cap = B * C * N
    indptr = torch.empty(B * C + 1, dtype=_I32, device=dev)
    batch_ids = torch.empty(cap, dtype=_I64, device=dev)
    camera_ids = torch.empty(cap, dtype=_I64, device=dev)
    gaussian_ids = torch.empty(cap, dtype=_I64, device=dev)
    radii = torch.empty(cap, 2, dtype=_I32, device=dev)
    means2d = torch.empty(cap, 2, dtype=_F32, device=dev)
    depths = torch.empty(cap, dtype=_F32, device=dev)
    conics = torch.empty(cap, 3, dtype=_F32, device=dev)
    comps = torch.empty(cap, dtype=_F32, device=dev) if calc_compensations else None
    row_of = torch.empty(cap, dtype=_I32, device=dev)
    row_opac = torch.empty(cap, dtype=_F32, device=dev)
    row_colors = torch.empty(cap, D, dtype=_F32, device=dev)
    if cap == 0:
        indptr.zero_()
        nnz = 0
    else:
        st = _stream(means)
        ws = torch.empty(query("gsplat_projection_packed_workspace_size", B, C, N),
                         dtype=torch.uint8, device=dev)
        # the kernel writes the visible count straight into pinned host
        # memory (device-accessible at the same address), so no copy kernel
        # sits on the stream between the projection and the colours
        nnz_host = torch.empty(1, dtype=_I64, pin_memory=True)
        call("gsplat_projection_packed_fwd", B, C, N, ptr(means), ptr(covars),
             ptr(quats), ptr(scales), ptr(opacities), ptr(viewmats), ptr(Ks),
             int(image_width), int(image_height), float(eps2d),
             float(near_plane), float(far_plane), float(radius_clip),
             int(camera_model), ptr(ws), ws.numel(), ptr(indptr),
             ptr(batch_ids), ptr(camera_ids), ptr(gaussian_ids), ptr(radii),
             ptr(means2d), ptr(depths), ptr(conics), ptr(comps), ptr(nnz_host),
             ptr(row_of), ptr(row_opac), st)
        copied = torch.cuda.Event()
        copied.record()
        I = B * C
        tile_first = isect is not None and (
            int(I).bit_length()
            + (int(isect["tile_width"]) * int(isect["tile_height"])).bit_length()) <= 32
        counted = None
        if sh_degree is None:
            call("gsplat_rows_gather", B, C, N, D, ptr(features), ptr(row_of),
                 ptr(row_colors), st)
        elif tile_first and B == 1:
            # the colours and the intersection's tile counts in one launch,
            # over the rows the projection counted on the device
            # (indptr[I]); the host's wait below then overlaps them both
            counted = {
                "tpg": torch.empty(cap, dtype=_I32, device=dev),
                "row_starts": torch.empty(cap + 1, dtype=_I64, device=dev),
                "records": torch.empty(cap, 8, dtype=_F32, device=dev),
                "ws": torch.empty(query("gsplat_isect_prepare_rows_workspace_size", cap),
                                  dtype=torch.uint8, device=dev),
            }
            call("gsplat_sh_rows_fwd_isect_count", B, C, N, K, int(sh_degree),
                 ptr(means), ptr(viewmats), ptr(features), ptr(row_of), ptr(row_colors),
                 cap, ptr(indptr[I:]), ptr(camera_ids) if I > 1 else None,
                 ptr(means2d), ptr(radii), ptr(depths), ptr(conics), ptr(row_opac),
                 int(isect["tile_size"]), int(isect["tile_width"]),
                 int(isect["tile_height"]), ptr(counted["ws"]), counted["ws"].numel(),
                 ptr(counted["tpg"]), ptr(counted["row_starts"]),
                 ptr(counted["records"]), st)
        else:
            call("gsplat_sh_rows_fwd", B, C, N, K, int(sh_degree), ptr(means),
                 ptr(viewmats), ptr(features), ptr(row_of), ptr(row_colors), st)
        copied.synchronize()
        nnz = int(nnz_host[0])
        if isect is not None and nnz > 0:
            ts, tw, th = isect["tile_size"], isect["tile_width"], isect["tile_height"]
            if tile_first:
                if I == 1:
                    img = None
                else:
                    img = (camera_ids[:nnz] if B == 1
                           else batch_ids[:nnz] * C + camera_ids[:nnz])
                if counted is not None:
                    state = isect_prepare_counted(
                        counted, means2d[:nnz], radii[:nnz], depths[:nnz], conics[:nnz],
                        row_opac[:nnz], img, nnz if I == 1 else 0, I, ts, tw, th)
                else:
                    state = isect_prepare_sorted(
                        means2d[:nnz], radii[:nnz], depths[:nnz], conics[:nnz],
                        row_opac[:nnz], img, nnz if I == 1 else 0, I, ts, tw, th,
                        torch.empty(nnz, dtype=_I32, device=dev))
                cap = isect_capacity(dev)
                if cap is not None:
                    isect_emit_sorted_queue(state, cap)
                isect["state"] = state
    return (
        indptr,
        batch_ids[:nnz],
        camera_ids[:nnz],
        gaussian_ids[:nnz],
        radii[:nnz],
        means2d[:nnz],
        depths[:nnz],
        conics[:nnz],
        comps[:nnz] if comps is not None else None,
        row_of,
        row_opac[:nnz],
        row_colors[:nnz],
    )


def projection_ewa_3dgs_packed_fwd(
    means: Tensor,
    covars: Optional[Tensor],
    quats: Optional[Tensor],
    scales: Optional[Tensor],
    opacities: Optional[Tensor],
    viewmats: Tensor,
    Ks: Tensor,
    image_width: int,
    image_height: int,
    eps2d: float,
    near_plane: float,
    far_plane: float,
    radius_clip: float,
    calc_compensations: bool,
    camera_model: int,
):
    return projection_packed_fwd_with_row_map(
        means, covars, quats, scales, opacities, viewmats, Ks, image_width,
        image_height, eps2d, near_plane, far_plane, radius_clip,
        calc_compensations, camera_model)[:9]


def projection_ewa_3dgs_packed_bwd(
    means: Tensor,
    covars: Optional[Tensor],
    quats: Optional[Tensor],
    scales: Optional[Tensor],
    viewmats: Tensor,
    Ks: Tensor,
    image_width: int,
    image_height: int,
    eps2d: float,
    camera_model: int,
    batch_ids: Tensor,
    camera_ids: Tensor,
    gaussian_ids: Tensor,
    conics: Tensor,
    compensations: Optional[Tensor],
    v_means2d: Tensor,
    v_depths: Tensor,
    v_conics: Tensor,
    v_compensations: Optional[Tensor],
    viewmats_requires_grad: bool,
    sparse_grad: bool,
):
    _check_proj_inputs(means, covars, quats, scales, None, viewmats, Ks)
    for t, n in ((batch_ids, "batch_ids"), (camera_ids, "camera_ids"),
                 (gaussian_ids, "gaussian_ids"), (conics, "conics"),
                 (v_means2d, "v_means2d"), (v_depths, "v_depths"),
                 (v_conics, "v_conics"), (compensations, "compensations"),
                 (v_compensations, "v_compensations")):
        check_input(t, n)
    batch_dims, B, C, N = _proj_dims(means, viewmats)
    nnz = batch_ids.shape[0]
    dev = means.device
    v_covars = v_quats = v_scales = None
    if sparse_grad:
        v_means = torch.empty(nnz, 3, dtype=_F32, device=dev)
        if covars is not None:
            v_covars = torch.empty(nnz, 6, dtype=_F32, device=dev)
        else:
            v_quats = torch.empty(nnz, 4, dtype=_F32, device=dev)
            v_scales = torch.empty(nnz, 3, dtype=_F32, device=dev)
    else:
        v_means = torch.zeros_like(means)
        if covars is not None:
            v_covars = torch.zeros_like(covars)
        else:
            v_quats = torch.zeros_like(quats)
            v_scales = torch.zeros_like(scales)
    v_viewmats = torch.zeros_like(viewmats) if viewmats_requires_grad else None
    call("gsplat_projection_packed_bwd", B, C, N, nnz, ptr(means), ptr(covars),
         ptr(quats), ptr(scales), ptr(viewmats), ptr(Ks), int(image_width),
         int(image_height), float(eps2d), int(camera_model), ptr(batch_ids),
         ptr(camera_ids), ptr(gaussian_ids), ptr(conics), ptr(compensations),
         ptr(v_means2d), ptr(v_depths), ptr(v_conics), ptr(v_compensations),
         int(bool(sparse_grad)), ptr(v_means), ptr(v_covars), ptr(v_quats),
         ptr(v_scales), ptr(v_viewmats), _stream(means))
    return v_means, v_covars, v_quats, v_scales, v_viewmats


def projection_packed_bwd_rows(
    means: Tensor,
    covars: Optional[Tensor],
    quats: Optional[Tensor],
    scales: Optional[Tensor],
    viewmats: Tensor,
    Ks: Tensor,
    image_width: int,
    image_height: int,
    eps2d: float,
    camera_model: int,
    row_of: Tensor,
    conics: Tensor,
    compensations: Optional[Tensor],
    v_means2d: Tensor,
    v_depths: Optional[Tensor],
    v_conics: Tensor,
    v_compensations: Optional[Tensor],
    viewmats_requires_grad: bool,
    v_row_opacities: Optional[Tensor] = None,
    v_means_add: Optional[Tensor] = None,
    stats: Optional[Tuple[Tensor, float, float, Tensor, Tensor]] = None,
):
    """Dense gradients of the packed projection from its row map ``row_of``
    (one pass driven by Gaussian; no zero fill, no atomics).  ``v_depths``
    may be None (zero gradient).  With ``v_row_opacities`` [nnz] it also
    returns v_opacities (each Gaussian's sum over its rows, shaped like
    ``means[..., 0]``); ``v_means_add`` (like ``means``) is added to v_means.
    ``stats`` = (row gradients [nnz, 2], scale_x, scale_y, grad2d [N],
    count [N]) also accumulates the densification statistics in the same pass
    (one batch only).
    Returns (v_means, v_covars, v_quats, v_scales, v_viewmats[, v_opacities])."""
    _check_proj_inputs(means, covars, quats, scales, None, viewmats, Ks)
    check_input(row_of, "row_of", _I32)
    for t, n in ((conics, "conics"), (v_means2d, "v_means2d"), (v_depths, "v_depths"),
                 (v_conics, "v_conics"), (compensations, "compensations"),
                 (v_compensations, "v_compensations")):
        check_input(t, n)
    batch_dims, B, C, N = _proj_dims(means, viewmats)
    v_means = torch.empty_like(means)
    v_covars = torch.empty_like(covars) if covars is not None else None
    v_quats = torch.empty_like(quats) if covars is None else None
    v_scales = torch.empty_like(scales) if covars is None else None
    v_viewmats = torch.zeros_like(viewmats) if viewmats_requires_grad else None
    check_input(v_row_opacities, "v_row_opacities", _F32)
    check_input(v_means_add, "v_means_add", _F32)
    if v_means_add is not None and v_means_add.shape != means.shape:
        raise RuntimeError("projection_packed_bwd_rows: v_means_add must be shaped like means")
    v_opacities = (torch.empty(means.shape[:-1], dtype=_F32, device=means.device)
                   if v_row_opacities is not None else None)
    if conics.shape[0] == 0:
        # no visible row: every gradient is zero (plus the added term); the
        # empty row buffers have no storage to hand to the kernel
        for t in (v_means, v_covars, v_quats, v_scales, v_opacities):
            if t is not None:
                t.zero_()
        if v_means_add is not None:
            v_means.copy_(v_means_add)
        if v_row_opacities is not None:
            return v_means, v_covars, v_quats, v_scales, v_viewmats, v_opacities
        return v_means, v_covars, v_quats, v_scales, v_viewmats
    args = [B, C, N, ptr(means), ptr(covars), ptr(quats), ptr(scales), ptr(viewmats),
            ptr(Ks), int(image_width), int(image_height), float(eps2d),
            int(camera_model), ptr(row_of), ptr(conics), ptr(compensations),
            ptr(v_means2d), ptr(v_depths), ptr(v_conics), ptr(v_compensations),
            ptr(v_means), ptr(v_covars), ptr(v_quats), ptr(v_scales), ptr(v_viewmats),
            ptr(v_row_opacities), ptr(v_opacities), ptr(v_means_add)]
    if stats is None:
        call("gsplat_projection_packed_bwd_rows", *args, _stream(means))
    else:
        grads, sx, sy, grad2d, count = stats
        check_input(grads, "stat_grads", _F32)
        check_input(grad2d, "grad2d", _F32)
        check_input(count, "count", _F32)
        if grads.shape != conics[:, :2].shape or grad2d.numel() != N or count.numel() != N:
            raise RuntimeError("projection_packed_bwd_rows: statistics buffers must be "
                               "[nnz, 2] row gradients and [N] accumulators")
        call("gsplat_projection_packed_bwd_rows_stats", *args, ptr(grads), float(sx),
             float(sy), ptr(grad2d), ptr(count), _stream(means))
    if v_row_opacities is not None:
        return v_means, v_covars, v_quats, v_scales, v_viewmats, v_opacities
    return v_means, v_covars, v_quats, v_scales, v_viewmats


def projection_packed_bwd_rows_sh(
    means: Tensor,
    covars: Optional[Tensor],
    quats: Optional[Tensor],
    scales: Optional[Tensor],
    viewmats: Tensor,
    Ks: Tensor,
    image_width: int,
    image_height: int,
    eps2d: float,
    camera_model: int,
    row_of: Tensor,
    conics: Tensor,
    compensations: Optional[Tensor],
    v_means2d: Tensor,
    v_depths: Optional[Tensor],
    v_conics: Tensor,
    v_compensations: Optional[Tensor],
    degree: int,
    coeffs: Tensor,
    v_colors: Tensor,
    v_row_opacities: Optional[Tensor] = None,
    stats: Optional[Tuple[Tensor, float, float, Tensor, Tensor]] = None,
):
    """projection_packed_bwd_rows (no view-matrix gradients) with the SH
    colours' backward of the same rows in the same launch
    (gsplat_projection_packed_bwd_rows_sh): the SH direction term is added to
    v_means inside the launch.  coeffs [..., N, K, 3] as the forward's,
    v_colors [nnz, 3].  Returns (v_means, v_covars, v_quats, v_scales,
    v_opacities or None, v_coeffs)."""
    _check_proj_inputs(means, covars, quats, scales, None, viewmats, Ks)
    check_input(row_of, "row_of", _I32)
    for t, n in ((conics, "conics"), (v_means2d, "v_means2d"), (v_depths, "v_depths"),
                 (v_conics, "v_conics"), (compensations, "compensations"),
                 (v_compensations, "v_compensations"), (coeffs, "coeffs"),
                 (v_colors, "v_colors")):
        check_input(t, n)
    check_input(v_row_opacities, "v_row_opacities", _F32)
    batch_dims, B, C, N = _proj_dims(means, viewmats)
    K = coeffs.shape[-2]
    if tuple(coeffs.shape) != tuple(batch_dims) + (N, K, 3) or v_colors.shape != conics.shape:
        raise RuntimeError("projection_packed_bwd_rows_sh: coeffs must be [..., N, K, 3] "
                           "and v_colors [nnz, 3]")
    if conics.shape[0] == 0:
        raise RuntimeError("projection_packed_bwd_rows_sh: no visible row (use the "
                           "separate backward passes)")
    v_means = torch.empty_like(means)
    v_covars = torch.empty_like(covars) if covars is not None else None
    v_quats = torch.empty_like(quats) if covars is None else None
    v_scales = torch.empty_like(scales) if covars is None else None
    v_coeffs = torch.empty_like(coeffs)
    v_opacities = (torch.empty(means.shape[:-1], dtype=_F32, device=means.device)
                   if v_row_opacities is not None else None)
    grads = grad2d = count = None
    sx = sy = 0.0
    if stats is not None:
        grads, sx, sy, grad2d, count = stats
        check_input(grads, "stat_grads", _F32)
        check_input(grad2d, "grad2d", _F32)
        check_input(count, "count", _F32)
        if grads.shape != conics[:, :2].shape or grad2d.numel() != N or count.numel() != N:
            raise RuntimeError("projection_packed_bwd_rows_sh: statistics buffers must be "
                               "[nnz, 2] row gradients and [N] accumulators")
    call("gsplat_projection_packed_bwd_rows_sh", B, C, N, ptr(means), ptr(covars),
         ptr(quats), ptr(scales), ptr(viewmats), ptr(Ks), int(image_width),
         int(image_height), float(eps2d), int(camera_model), ptr(row_of), ptr(conics),
         ptr(compensations), ptr(v_means2d), ptr(v_depths), ptr(v_conics),
         ptr(v_compensations), ptr(v_means), ptr(v_covars), ptr(v_quats), ptr(v_scales),
         ptr(v_row_opacities), ptr(v_opacities), ptr(grads), float(sx), float(sy),
         ptr(grad2d), ptr(count), K, int(degree), ptr(coeffs), ptr(v_colors),
         ptr(v_coeffs), _stream(means))
    return v_means, v_covars, v_quats, v_scales, v_opacities, v_coeffs


# --------------------------------------------------------------------------
# Packed rows driven by Gaussian (replace the gathers / index_put scatters of
# the packed path, rendering.py:95-213, 782, 845-873)
# --------------------------------------------------------------------------
def sh_rows_fwd(degree: int, means: Tensor, viewmats: Tensor, coeffs: Tensor,
                row_of: Tensor, nnz: int, fill: Optional[float] = None) -> Tensor:
    """colors [nnz, 3] = max(SH(normalize(mean - centre)) + 0.5, 0) for every
    packed row, centre = -R^T t of the camera; means [B, N, 3], viewmats
    [B, C, 4, 4], coeffs [B, N, K, 3].  Rows that no entry of row_of names
    hold ``fill`` (left unset when it is None)."""
    for t, n in ((means, "means"), (viewmats, "viewmats"), (coeffs, "coeffs")):
        check_input(t, n, _F32)
    check_input(row_of, "row_of", _I32)
    B, N = means.shape[0], means.shape[1]
    C = viewmats.shape[1]
    K = coeffs.shape[-2]
    colors = (torch.empty(nnz, 3, dtype=_F32, device=means.device) if fill is None
              else torch.full((nnz, 3), fill, dtype=_F32, device=means.device))
    if nnz == 0:
        return colors
    call("gsplat_sh_rows_fwd", B, C, N, K, int(degree), ptr(means), ptr(viewmats),
         ptr(coeffs), ptr(row_of), ptr(colors), _stream(means))
    return colors


def sh_rows_bwd(degree: int, means: Tensor, viewmats: Tensor, coeffs: Tensor,
                row_of: Tensor, v_colors: Tensor) -> Tuple[Tensor, Tensor]:
    check_input(v_colors, "v_colors", _F32)
    B, N = means.shape[0], means.shape[1]
    C = viewmats.shape[1]
    K = coeffs.shape[-2]
    v_coeffs = torch.empty_like(coeffs)
    v_means = torch.empty_like(means)
    if v_colors.shape[0] == 0:  # no visible row: zero gradients
        return v_coeffs.zero_(), v_means.zero_()
    call("gsplat_sh_rows_bwd", B, C, N, K, int(degree), ptr(means), ptr(viewmats),
         ptr(coeffs), ptr(row_of), ptr(v_colors), ptr(v_coeffs), ptr(v_means),
         _stream(means))
    return v_coeffs, v_means


def rows_gather(src: Tensor, row_of: Tensor, C: int, nnz: int) -> Tensor:
    """out [nnz, F] with out[row_of[b, c, g]] = src[b, g]; src [B, N, F]."""
    check_input(src, "src", _F32)
    check_input(row_of, "row_of", _I32)
    B, N, F = src.shape
    out = torch.empty(nnz, F, dtype=_F32, device=src.device)
    if nnz == 0:
        return out
    call("gsplat_rows_gather", B, int(C), N, F, ptr(src), ptr(row_of), ptr(out),
         _stream(src))
    return out


def rows_scatter_sum(v_out: Tensor, row_of: Tensor, B: int, C: int, N: int) -> Tensor:
    """v_src [B, N, F]: per Gaussian, the sum of its rows' gradients."""
    check_input(v_out, "v_out", _F32)
    F = v_out.shape[-1]
    v_src = torch.empty(B, N, F, dtype=_F32, device=v_out.device)
    if v_out.shape[0] == 0:  # no visible row: zero gradients
        return v_src.zero_()
    call("gsplat_rows_scatter_sum", int(B), int(C), int(N), F, ptr(row_of),
         ptr(v_out), ptr(v_src), _stream(v_out))
    return v_src


# --------------------------------------------------------------------------
# Tile intersection  (Intersect.cpp:33-164, 320-337)
# --------------------------------------------------------------------------
def intersect_tile(
    means2d: Tensor,
    radii: Tensor,
    depths: Tensor,
    conics: Optional[Tensor],
    opacities: Optional[Tensor],
    image_ids: Optional[Tensor],
    gaussian_ids: Optional[Tensor],
    I: int,
    tile_size: int,
    tile_width: int,
    tile_height: int,
    sort: bool,
    segmented: bool,
) -> Tuple[Tensor, Tensor, Tensor]:
    check_input(means2d, "means2d", _F32)
    check_input(radii, "radii", _I32)
    check_input(depths, "depths", _F32)
    check_input(conics, "conics", _F32)
    check_input(opacities, "opacities", _F32)
    packed = means2d.dim() == 2
    if packed:
        if image_ids is None or gaussian_ids is None:
            raise RuntimeError(
                "When packed is set, image_ids and gaussian_ids must be provided.")
        check_input(image_ids, "image_ids", _I64)
        check_input(gaussian_ids, "gaussian_ids", _I64)
    n = means2d.numel() // 2
    N = 0 if packed else means2d.shape[-2]
    n_tiles = int(tile_width) * int(tile_height)
    tile_n_bits = n_tiles.bit_length()
    image_n_bits = int(I).bit_length()
    if image_n_bits + tile_n_bits > 32:
        raise RuntimeError("intersect_tile: image and tile ids need more than 32 bits")
    dev = means2d.device
    tiles_per_gauss = torch.empty(depths.shape, dtype=_I32, device=dev)
    if n == 0:
        return (tiles_per_gauss, torch.empty(0, dtype=_I64, device=dev),
                torch.empty(0, dtype=_I32, device=dev))
    st = _stream(means2d)
    img = image_ids if packed else None
    if packed and int(I) == 1:
        # one image: every row's image id is 0, which the dense layout with
        # N = n gives (row // n) without reading the ids
        img, N = None, n
    if sort:
        # Intersections emitted in row order, stably sorted on the image|tile
        # bits, then every tile's rows stably sorted on their depth bits: the
        # reference's full-key order (a per-image segmented sort,
        # segmented=True, is the same order because the image id occupies
        # the top key bits).
        state = isect_prepare_sorted(means2d, radii, depths, conics, opacities, img,
                                     N, I, tile_size, tile_width, tile_height,
                                     tiles_per_gauss)
        return isect_emit_sorted(state)[:3]
    cum = torch.empty(n, dtype=_I64, device=dev)
    ws = torch.empty(query("gsplat_isect_count_workspace_size", n),
                     dtype=torch.uint8, device=dev)
    call("gsplat_isect_count", n, N, ptr(img), ptr(means2d), ptr(radii),
         ptr(conics), ptr(opacities), int(tile_size), int(tile_width),
         int(tile_height), ptr(ws), ws.numel(), ptr(tiles_per_gauss), ptr(cum), st)
    n_isects = int(cum[-1].item())
    isect_ids = torch.empty(n_isects, dtype=_I64, device=dev)
    flatten_ids = torch.empty(n_isects, dtype=_I32, device=dev)
    if n_isects == 0:
        return tiles_per_gauss, isect_ids, flatten_ids
    call("gsplat_isect_emit", n, N, int(I), ptr(img), ptr(means2d), ptr(radii),
         ptr(depths), ptr(conics), ptr(opacities), int(tile_size),
         int(tile_width), int(tile_height), ptr(cum), ptr(isect_ids),
         ptr(flatten_ids), st)
    return tiles_per_gauss, isect_ids, flatten_ids


# Intersection count of the last sorted intersection per device: the next
# call queues its emission for this many plus 1/16 (and 4096) before the
# host knows its own count.
_ISECT_LAST = {}


def isect_capacity(device: torch.device) -> Optional[int]:
    """Capacity for a device-counted emission (None before the first count)."""
    last = _ISECT_LAST.get(device.index)
    return None if last is None else last + last // 16 + 4096


def isect_emit_sorted_queue(state, capacity: int) -> None:
    """Queues the second half of the sorted intersection behind the first
    with the count read on the device (gsplat_isect_emit_tiles_dev), into
    buffers of ``capacity`` entries; ``isect_emit_sorted`` then only checks
    the count against the capacity."""
    dev = state["means2d"].device
    isect_ids = torch.empty(capacity, dtype=_I64, device=dev)
    flatten_ids = torch.empty(capacity, dtype=_I32, device=dev)
    ts, tw, th = state["tile"]
    offsets = torch.empty((state["I"], th, tw), dtype=_I32, device=dev)
    ews = torch.empty(query("gsplat_isect_emit_tiles_workspace_size", capacity),
                      dtype=torch.uint8, device=dev)
    call("gsplat_isect_emit_tiles_dev", state["n"], state["N"], state["I"],
         ptr(state["img"]), ptr(state["means2d"]), ptr(state["radii"]),
         ptr(state["depths"]), ptr(state["conics"]), ptr(state["opacities"]), ts, tw,
         th, ptr(state["row_starts"]), ptr(state["records"]), int(capacity), ptr(ews),
         ews.numel(), ptr(isect_ids), ptr(flatten_ids), ptr(offsets),
         _stream(state["means2d"]))
    state["queued"] = (int(capacity), isect_ids, flatten_ids, offsets)


def isect_prepare_sorted(means2d, radii, depths, conics, opacities, img, N, I,
                         tile_size, tile_width, tile_height, tiles_per_gauss):
    """First half of the sorted intersection of n > 0 rows (inputs checked by
    the caller): the tile counts, the rows' first slots in row order and
    their sweep records (gsplat_isect_prepare_rows).  The intersection count
    goes to a pinned host word behind an event, so the caller can queue or
    do other work before ``isect_emit_sorted`` waits for it."""
    n = means2d.numel() // 2
    dev = means2d.device
    st = _stream(means2d)
    state = {
        "n": n, "N": N, "I": int(I), "img": img, "means2d": means2d, "radii": radii,
        "depths": depths, "conics": conics, "opacities": opacities,
        "tile": (int(tile_size), int(tile_width), int(tile_height)),
        "tiles_per_gauss": tiles_per_gauss,
        "row_starts": torch.empty(n + 1, dtype=_I64, device=dev),
        "records": torch.empty(n, 8, dtype=_F32, device=dev),
    }
    # the count goes straight into pinned host memory (no copy kernel)
    host = torch.empty(1, dtype=_I64, pin_memory=True)
    ws = torch.empty(query("gsplat_isect_prepare_rows_workspace_size", n),
                     dtype=torch.uint8, device=dev)
    call("gsplat_isect_prepare_rows", n, N, ptr(img), ptr(means2d), ptr(radii),
         ptr(depths), ptr(conics), ptr(opacities), int(tile_size),
         int(tile_width), int(tile_height), ptr(ws), ws.numel(),
         ptr(tiles_per_gauss), ptr(state["row_starts"]), ptr(state["records"]),
         ptr(host), st)
    ev = torch.cuda.Event()
    ev.record()
    state["total"] = (host, ev)
    return state


def isect_prepare_counted(counted, means2d, radii, depths, conics, opacities, img, N,
                          I, tile_size, tile_width, tile_height):
    """isect_prepare_sorted's state for n > 0 rows whose tile counts, count
    prefixes and sweep records gsplat_sh_rows_fwd_isect_count already wrote
    into the capacity-sized buffers of ``counted``: only the row starts and
    the intersection count remain (gsplat_isect_row_starts)."""
    n = means2d.numel() // 2
    state = {
        "n": n, "N": N, "I": int(I), "img": img, "means2d": means2d, "radii": radii,
        "depths": depths, "conics": conics, "opacities": opacities,
        "tile": (int(tile_size), int(tile_width), int(tile_height)),
        "tiles_per_gauss": counted["tpg"][:n],
        "row_starts": counted["row_starts"][:n + 1],
        "records": counted["records"][:n],
    }
    host = torch.empty(1, dtype=_I64, pin_memory=True)
    call("gsplat_isect_row_starts", n, ptr(counted["ws"]), counted["ws"].numel(),
         ptr(state["row_starts"]), ptr(host), _stream(means2d))
    ev = torch.cuda.Event()
    ev.record()
    state["total"] = (host, ev)
    return state


def isect_emit_sorted(state):
    """Second half: waits for the intersection count, then emits the
    intersections in row order, sorts them on the image|tile bits and every
    tile's rows on their depth bits (gsplat_isect_emit_tiles).  Returns
    (tiles_per_gauss, isect_ids, flatten_ids, isect_offsets [I, th, tw])."""
    host, ev = state["total"]
    ev.synchronize()
    n_isects = int(host[0])
    dev = state["means2d"].device
    _ISECT_LAST[dev.index] = n_isects
    queued = state.get("queued")
    if queued is not None and n_isects <= queued[0]:
        return (state["tiles_per_gauss"], queued[1][:n_isects], queued[2][:n_isects],
                queued[3])
    # no queued emission, or more intersections than it had room for (its
    # output is dropped): emit with the exact count
    ts, tw, th = state["tile"]
    isect_ids = torch.empty(n_isects, dtype=_I64, device=dev)
    flatten_ids = torch.empty(n_isects, dtype=_I32, device=dev)
    offsets = torch.empty((state["I"], th, tw), dtype=_I32, device=dev)
    ews = torch.empty(query("gsplat_isect_emit_tiles_workspace_size", n_isects),
                      dtype=torch.uint8, device=dev)
    call("gsplat_isect_emit_tiles", state["n"], state["N"], state["I"],
         ptr(state["img"]), ptr(state["means2d"]), ptr(state["radii"]),
         ptr(state["depths"]), ptr(state["conics"]), ptr(state["opacities"]), ts, tw,
         th, ptr(state["row_starts"]), ptr(state["records"]), n_isects, ptr(ews),
         ews.numel(), ptr(isect_ids), ptr(flatten_ids), ptr(offsets),
         _stream(state["means2d"]))
    return state["tiles_per_gauss"], isect_ids, flatten_ids, offsets


def intersect_offset(isect_ids: Tensor, I: int, tile_width: int, tile_height: int) -> Tensor:
    check_input(isect_ids, "isect_ids", _I64)
    offsets = torch.empty((int(I), int(tile_height), int(tile_width)), dtype=_I32,
                          device=isect_ids.device)
    call("gsplat_isect_offsets", isect_ids.numel(), ptr(isect_ids), int(I),
         int(tile_width), int(tile_height), ptr(offsets), _stream(isect_ids))
    return offsets


# --------------------------------------------------------------------------
# Rasterizer  (Rasterization.cpp:42-214)
# --------------------------------------------------------------------------
def _raster_common(means2d, conics, colors, opacities, backgrounds, masks,
                   tile_offsets, flatten_ids):
    check_input(means2d, "means2d", _F32)
    check_input(conics, "conics", _F32)
    check_input(colors, "colors", _F32)
    check_input(opacities, "opacities", _F32)
    check_input(backgrounds, "backgrounds", _F32)
    check_input(masks, "masks", torch.bool)
    check_input(tile_offsets, "tile_offsets", _I32)
    check_input(flatten_ids, "flatten_ids", _I32)
    image_dims = tuple(tile_offsets.shape[:-2])
    tile_height, tile_width = tile_offsets.shape[-2:]
    I = _prod(image_dims)
    n_rows = means2d.numel() // 2
    return image_dims, I, n_rows, tile_width, tile_height


def rasterize_fwd_with_transmittance(
    means2d: Tensor,
    conics: Tensor,
    colors: Tensor,
    opacities: Tensor,
    backgrounds: Optional[Tensor],
    masks: Optional[Tensor],
    image_width: int,
    image_height: int,
    tile_size: int,
    tile_offsets: Tensor,
    flatten_ids: Tensor,
) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """Forward rasterizer that also returns the final transmittance T of every
    pixel ([..., H, W] float32); the autograd wrapper hands T to the backward
    instead of re-deriving it as 1 - alpha."""
    image_dims, I, n_rows, tw, th = _raster_common(
        means2d, conics, colors, opacities, backgrounds, masks, tile_offsets,
        flatten_ids)
    channels = colors.shape[-1]
    dev = means2d.device
    H, W = int(image_height), int(image_width)
    renders = torch.empty(image_dims + (H, W, channels), dtype=_F32, device=dev)
    alphas = torch.empty(image_dims + (H, W, 1), dtype=_F32, device=dev)
    last_ids = torch.empty(image_dims + (H, W), dtype=_I32, device=dev)
    transmittance = torch.empty(image_dims + (H, W), dtype=_F32, device=dev)
    call("gsplat_rasterize_fwd", I, n_rows, flatten_ids.numel(), channels,
         ptr(means2d), ptr(conics), ptr(colors), ptr(opacities),
         ptr(backgrounds), ptr(masks), W, H, int(tile_size), tw, th,
         ptr(tile_offsets), ptr(flatten_ids), ptr(renders), ptr(alphas),
         ptr(last_ids), ptr(transmittance), _stream(means2d))
    return renders, alphas, last_ids, transmittance


class RasterReplay:
    """What ``rasterize_fwd_replay`` keeps for ``rasterize_bwd_replay``: the
    replay records and unit list (``records``), the zeroed accumulators of
    the backward (``accum``, used once, or None) and the expected-depth
    channel of the render (``expected_depth`` [..., H, W], or None) with its
    index ``channel`` (-1 for none)."""

    __slots__ = ("records", "accum", "expected_depth", "channel")

    def __init__(self, records, accum, expected_depth, channel):
        self.records = records
        self.accum = accum
        self.expected_depth = expected_depth
        self.channel = channel


# Largest replay workspace (bytes) one rasterizer call may allocate.  The
# records take 16 (1 + C) bytes per intersection for C channels (a record of
# T and the C colour sums for each of a tile's pixels at every 64th
# intersection of its range), allocated for the whole range although only the
# boundaries a pixel is still active at are written.  Above this budget the
# forward keeps no replay state and the backward replays whole tiles from the
# final transmittance (gsplat_rasterize_bwd), as the reference does.
replay_budget_bytes = 8 << 30


def rasterize_replay_bytes(image_dims_numel: int, tile_width: int, tile_height: int,
                           tile_size: int, n_isects: int, channels: int) -> int:
    """Bytes of the replay workspace ``rasterize_fwd_replay`` allocates."""
    return query("gsplat_rasterize_replay_size", image_dims_numel, tile_width,
                 tile_height, int(tile_size), n_isects, channels)


def rasterize_fwd_replay(
    means2d: Tensor,
    conics: Tensor,
    colors: Tensor,
    opacities: Tensor,
    backgrounds: Optional[Tensor],
    masks: Optional[Tensor],
    image_width: int,
    image_height: int,
    tile_size: int,
    tile_offsets: Tensor,
    flatten_ids: Tensor,
    expected_depth_channel: int = -1,
    absgrad: Optional[bool] = None,
    color_last: Optional[Tensor] = None,
):
    """``rasterize_fwd_with_transmittance`` that also keeps the replay state of
    ``rasterize_bwd_replay`` (per-pixel records at every batch boundary of a
    tile and the list of replay units), returned as a ``RasterReplay`` fifth
    output.  With ``expected_depth_channel`` >= 0 that channel of the render
    is divided by max(alpha, 1e-10) (rendering.py:1259-1267) and kept in the
    state for the backward.  With ``absgrad`` not None the launch also
    zero-fills the accumulators of ``rasterize_bwd_replay``.  With
    ``color_last`` [..., n] the render has one channel more than ``colors``,
    its last one taken from ``color_last`` (a depth channel, without
    concatenating it to the colours)."""
    image_dims, I, n_rows, tw, th = _raster_common(
        means2d, conics, colors, opacities, backgrounds, masks, tile_offsets,
        flatten_ids)
    channels = _raster_channels(colors, color_last, n_rows)
    dev = means2d.device
    H, W = int(image_height), int(image_width)
    renders = torch.empty(image_dims + (H, W, channels), dtype=_F32, device=dev)
    alphas = torch.empty(image_dims + (H, W, 1), dtype=_F32, device=dev)
    last_ids = torch.empty(image_dims + (H, W), dtype=_I32, device=dev)
    transmittance = torch.empty(image_dims + (H, W), dtype=_F32, device=dev)
    n_isects = flatten_ids.numel()
    records = torch.empty(rasterize_replay_bytes(I, tw, th, tile_size, n_isects, channels),
                          dtype=torch.uint8, device=dev)
    accum = None
    if absgrad is not None:
        accum = torch.empty(_bwd_accum_words(means2d, conics, colors, opacities, absgrad,
                                             color_last),
                            dtype=_F32, device=dev)
    ed = None
    if expected_depth_channel >= 0:
        ed = torch.empty(image_dims + (H, W), dtype=_F32, device=dev)
    call("gsplat_rasterize_fwd_replay", I, n_rows, n_isects, channels,
         ptr(means2d), ptr(conics), ptr(colors), ptr(color_last), ptr(opacities),
         ptr(backgrounds), ptr(masks), W, H, int(tile_size), tw, th,
         ptr(tile_offsets), ptr(flatten_ids), ptr(renders), ptr(alphas),
         ptr(last_ids), ptr(transmittance), ptr(records), records.numel(),
         int(expected_depth_channel), ptr(ed), ptr(accum),
         0 if accum is None else accum.numel(), _stream(means2d))
    return (renders, alphas, last_ids, transmittance,
            RasterReplay(records, accum, ed, int(expected_depth_channel)))


def _bwd_accum_words(means2d, conics, colors, opacities, absgrad: bool,
                     color_last=None) -> int:
    """Floats of the backward's accumulators: v_means2d, v_conics, v_colors,
    v_opacities (, v_means2d_abs) (, v_color_last) and the one-word unit
    counter."""
    n = means2d.numel() + conics.numel() + colors.numel() + opacities.numel() + 1
    n += color_last.numel() if color_last is not None else 0
    return n + (means2d.numel() if absgrad else 0)


def _raster_channels(colors: Tensor, color_last: Optional[Tensor], n_rows: int) -> int:
    """Channels of the render: those of ``colors``, plus one for a separate
    last channel ``color_last`` (one value per row)."""
    if color_last is None:
        return colors.shape[-1]
    check_input(color_last, "color_last", _F32)
    if color_last.numel() != n_rows or colors.numel() != n_rows * colors.shape[-1]:
        raise RuntimeError("color_last must hold one value per row of colors")
    return colors.shape[-1] + 1


def rasterize_to_pixels_3dgs_fwd(
    means2d: Tensor,
    conics: Tensor,
    colors: Tensor,
    opacities: Tensor,
    backgrounds: Optional[Tensor],
    masks: Optional[Tensor],
    image_width: int,
    image_height: int,
    tile_size: int,
    tile_offsets: Tensor,
    flatten_ids: Tensor,
) -> Tuple[Tensor, Tensor, Tensor]:
    image_dims, I, n_rows, tw, th = _raster_common(
        means2d, conics, colors, opacities, backgrounds, masks, tile_offsets,
        flatten_ids)
    channels = colors.shape[-1]
    dev = means2d.device
    H, W = int(image_height), int(image_width)
    renders = torch.empty(image_dims + (H, W, channels), dtype=_F32, device=dev)
    alphas = torch.empty(image_dims + (H, W, 1), dtype=_F32, device=dev)
    last_ids = torch.empty(image_dims + (H, W), dtype=_I32, device=dev)
    call("gsplat_rasterize_fwd", I, n_rows, flatten_ids.numel(), channels,
         ptr(means2d), ptr(conics), ptr(colors), ptr(opacities),
         ptr(backgrounds), ptr(masks), W, H, int(tile_size), tw, th,
         ptr(tile_offsets), ptr(flatten_ids), ptr(renders), ptr(alphas),
         ptr(last_ids), None, _stream(means2d))
    return renders, alphas, last_ids


def rasterize_to_pixels_3dgs_bwd(
    means2d: Tensor,
    conics: Tensor,
    colors: Tensor,
    opacities: Tensor,
    backgrounds: Optional[Tensor],
    masks: Optional[Tensor],
    image_width: int,
    image_height: int,
    tile_size: int,
    tile_offsets: Tensor,
    flatten_ids: Tensor,
    render_alphas: Tensor,
    last_ids: Tensor,
    v_render_colors: Tensor,
    v_render_alphas: Optional[Tensor],
    absgrad: bool,
    render_transmittance: Optional[Tensor] = None,
):
    """``render_transmittance`` (not part of the reference schema) is the
    forward's per-pixel T; without it T is taken as 1 - render_alphas.
    ``v_render_alphas`` may be None (zero)."""
    image_dims, I, n_rows, tw, th = _raster_common(
        means2d, conics, colors, opacities, backgrounds, masks, tile_offsets,
        flatten_ids)
    check_input(render_alphas, "render_alphas", _F32)
    check_input(last_ids, "last_ids", _I32)
    check_input(v_render_colors, "v_render_colors", _F32)
    check_input(v_render_alphas, "v_render_alphas", _F32)
    check_input(render_transmittance, "render_transmittance", _F32)
    channels = colors.shape[-1]
    # the kernel accumulates with atomics: one zero fill for every
    # accumulator, handed out as disjoint views, plus the zeroed tile counter
    # its workgroups take their tiles from
    likes = [means2d, conics, colors, opacities] + ([means2d] if absgrad else [])
    sizes = [t.numel() for t in likes] + [1]
    parts = torch.zeros(sum(sizes), dtype=_F32, device=means2d.device).split(sizes)
    v_means2d, v_conics, v_colors, v_opacities = (
        parts[k].view(likes[k].shape) for k in range(4))
    v_means2d_abs = parts[4].view(means2d.shape) if absgrad else None
    tile_counter = parts[-1]
    call("gsplat_rasterize_bwd", I, n_rows, flatten_ids.numel(), channels,
         ptr(means2d), ptr(conics), ptr(colors), ptr(opacities),
         ptr(backgrounds), ptr(masks), int(image_width), int(image_height),
         int(tile_size), tw, th, ptr(tile_offsets), ptr(flatten_ids),
         ptr(render_alphas), ptr(render_transmittance), ptr(last_ids),
         ptr(v_render_colors),
         ptr(v_render_alphas), ptr(v_means2d_abs), ptr(v_means2d),
         ptr(v_conics), ptr(v_colors), ptr(v_opacities), ptr(tile_counter),
         _stream(means2d))
    return v_means2d_abs, v_means2d, v_conics, v_colors, v_opacities


def rasterize_bwd_replay(
    means2d: Tensor,
    conics: Tensor,
    colors: Tensor,
    opacities: Tensor,
    backgrounds: Optional[Tensor],
    masks: Optional[Tensor],
    image_width: int,
    image_height: int,
    tile_size: int,
    tile_offsets: Tensor,
    flatten_ids: Tensor,
    render_transmittance: Tensor,
    last_ids: Tensor,
    replay: RasterReplay,
    v_render_colors: Tensor,
    v_render_alphas: Optional[Tensor],
    absgrad: bool,
    color_last: Optional[Tensor] = None,
):
    """``rasterize_to_pixels_3dgs_bwd`` from the state of
    ``rasterize_fwd_replay`` on the same inputs: the replay runs one unit per
    forward batch instead of one per tile.  With the forward's expected-depth
    channel the colour gradient of that channel is taken through its division
    by the alpha.  The state's zeroed accumulators are used once; a second
    backward allocates fresh zeros.  With ``color_last`` (as in the forward)
    a sixth output holds its gradient."""
    image_dims, I, n_rows, tw, th = _raster_common(
        means2d, conics, colors, opacities, backgrounds, masks, tile_offsets,
        flatten_ids)
    check_input(render_transmittance, "render_transmittance", _F32)
    check_input(last_ids, "last_ids", _I32)
    check_input(replay.records, "replay records", torch.uint8)
    check_input(v_render_colors, "v_render_colors", _F32)
    check_input(v_render_alphas, "v_render_alphas", _F32)
    check_input(replay.expected_depth, "expected_depth", _F32)
    if replay.channel >= 0 and (replay.expected_depth is None or
                                replay.expected_depth.shape != v_render_colors.shape[:-1]):
        raise RuntimeError("the expected-depth channel needs the forward's expected depth")
    channels = _raster_channels(colors, color_last, n_rows)
    likes = ([means2d, conics, colors, opacities] + ([means2d] if absgrad else [])
             + ([color_last] if color_last is not None else []))
    sizes = [t.numel() for t in likes] + [1]
    accum, replay.accum = replay.accum, None
    if accum is not None:
        check_input(accum, "accum", _F32)
        if accum.numel() != sum(sizes):
            raise RuntimeError("accum does not match the backward's accumulators")
        buf = accum
    else:
        buf = torch.zeros(sum(sizes), dtype=_F32, device=means2d.device)
    parts = buf.split(sizes)
    v_means2d, v_conics, v_colors, v_opacities = (
        parts[k].view(likes[k].shape) for k in range(4))
    v_means2d_abs = parts[4].view(means2d.shape) if absgrad else None
    v_color_last = (parts[len(likes) - 1].view(color_last.shape)
                    if color_last is not None else None)
    tile_counter = parts[-1]
    call("gsplat_rasterize_bwd_replay", I, n_rows, flatten_ids.numel(), channels,
         ptr(means2d), ptr(conics), ptr(colors), ptr(color_last), ptr(opacities),
         ptr(backgrounds), ptr(masks), int(image_width), int(image_height),
         int(tile_size), tw, th, ptr(tile_offsets), ptr(flatten_ids),
         ptr(render_transmittance), ptr(last_ids), ptr(v_render_colors),
         ptr(v_render_alphas), ptr(v_means2d_abs), ptr(v_means2d),
         ptr(v_conics), ptr(v_colors), ptr(v_color_last), ptr(v_opacities),
         ptr(tile_counter), ptr(replay.records), replay.records.numel(),
         ptr(replay.expected_depth), replay.channel, _stream(means2d))
    if color_last is not None:
        return v_means2d_abs, v_means2d, v_conics, v_colors, v_opacities, v_color_last
    return v_means2d_abs, v_means2d, v_conics, v_colors, v_opacities


# --------------------------------------------------------------------------
# Covariance / precision  (QuatScaleToCovar.cpp:37-110)
# --------------------------------------------------------------------------
def quat_scale_to_covar_preci_fwd(quats: Tensor, scales: Tensor, compute_covar: bool,
                                  compute_preci: bool, triu: bool):
    check_input(quats, "quats", _F32)
    check_input(scales, "scales", _F32)
    if quats.shape[-1] != 4 or scales.shape[:-1] != quats.shape[:-1] \
            or scales.shape[-1] != 3:
        raise RuntimeError("quats must be [..., 4] and scales [..., 3]")
    N = quats.numel() // 4
    out_shape = tuple(quats.shape[:-1]) + ((6,) if triu else (3, 3))
    covars = torch.empty(out_shape, dtype=_F32, device=quats.device) \
        if compute_covar else None
    precis = torch.empty(out_shape, dtype=_F32, device=quats.device) \
        if compute_preci else None
    call("gsplat_quat_scale_to_covar_preci_fwd", N, ptr(quats), ptr(scales),
         1 if triu else 0, ptr(covars), ptr(precis), _stream(quats))
    return covars, precis


def quat_scale_to_covar_preci_bwd(quats: Tensor, scales: Tensor, triu: bool,
                                  v_covars: Optional[Tensor],
                                  v_precis: Optional[Tensor]):
    check_input(quats, "quats", _F32)
    check_input(scales, "scales", _F32)
    check_input(v_covars, "v_covars", _F32)
    check_input(v_precis, "v_precis", _F32)
    N = quats.numel() // 4
    per = 6 if triu else 9
    for t, name in ((v_covars, "v_covars"), (v_precis, "v_precis")):
        if t is not None and t.numel() != N * per:
            raise RuntimeError(f"{name} must hold {per} values per Gaussian")
    v_quats = torch.empty_like(quats)
    v_scales = torch.empty_like(scales)
    call("gsplat_quat_scale_to_covar_preci_bwd", N, ptr(quats), ptr(scales),
         1 if triu else 0, ptr(v_covars), ptr(v_precis), ptr(v_quats),
         ptr(v_scales), _stream(quats))
    return v_quats, v_scales


# --------------------------------------------------------------------------
# Rasterize to indices  (Rasterization.cpp:216-308)
# --------------------------------------------------------------------------
def rasterize_to_indices_3dgs(range_start: int, range_end: int, transmittances: Tensor,
                              means2d: Tensor, conics: Tensor, opacities: Tensor,
                              image_width: int, image_height: int, tile_size: int,
                              tile_offsets: Tensor, flatten_ids: Tensor):
    for t, n, dt in ((transmittances, "transmittances", _F32), (means2d, "means2d", _F32),
                     (conics, "conics", _F32), (opacities, "opacities", _F32),
                     (tile_offsets, "tile_offsets", _I32),
                     (flatten_ids, "flatten_ids", _I32)):
        check_input(t, n, dt)
    N = means2d.shape[-2]
    I = means2d.numel() // (2 * N) if N > 0 else 0
    tile_height, tile_width = tile_offsets.shape[-2:]
    H, W = int(image_height), int(image_width)
    n_isects = flatten_ids.numel()
    dev = means2d.device
    if n_isects == 0 or I == 0:
        empty = torch.empty(0, dtype=torch.int64, device=dev)
        return empty, empty.clone()
    if transmittances.numel() != I * H * W:
        raise RuntimeError("transmittances must be [..., image_height, image_width]")
    n_pix = I * H * W
    cnts = torch.empty(n_pix, dtype=_I32, device=dev)
    starts = torch.empty(n_pix, dtype=_I32, device=dev)
    total = torch.empty(1, dtype=torch.int64, device=dev)
    ws = torch.empty(query("gsplat_rasterize_to_indices_workspace_size", n_pix),
                     dtype=torch.uint8, device=dev)
    args = (int(range_start), int(min(range_end, 2 ** 62)), I, N, n_isects,
            ptr(transmittances), ptr(means2d), ptr(conics), ptr(opacities), W, H,
            int(tile_size), int(tile_width), int(tile_height), ptr(tile_offsets),
            ptr(flatten_ids))
    call("gsplat_rasterize_to_indices_count", *args, ptr(cnts), ptr(starts),
         ptr(total), ptr(ws), ws.numel(), _stream(means2d))
    n_elems = int(total.item())
    gaussian_ids = torch.empty(n_elems, dtype=torch.int64, device=dev)
    pixel_ids = torch.empty(n_elems, dtype=torch.int64, device=dev)
    if n_elems:
        call("gsplat_rasterize_to_indices_write", *args, ptr(starts),
             ptr(gaussian_ids), ptr(pixel_ids), _stream(means2d))
    return gaussian_ids, pixel_ids


# --------------------------------------------------------------------------
# Densification statistics  (strategy/default.py:218-268)
# --------------------------------------------------------------------------
def grad2d_stats(grads: Tensor, gaussian_ids: Optional[Tensor],
                 radii: Optional[Tensor], n_gaussians: int, scale_x: float,
                 scale_y: float, grad2d: Tensor, count: Tensor) -> None:
    """grad2d[g] += ||grads[r] * (scale_x, scale_y)||, count[g] += 1 for every
    visible row r: packed rows (``gaussian_ids``) or dense rows [..., N]
    counted where both ``radii`` are > 0."""
    check_input(grads, "grads", _F32)
    check_input(gaussian_ids, "gaussian_ids", torch.int64)
    check_input(radii, "radii", _I32)
    check_input(grad2d, "grad2d", _F32)
    check_input(count, "count", _F32)
    if grads.shape[-1] != 2:
        raise RuntimeError("grads must end in a dimension of 2")
    n_rows = grads.numel() // 2
    if grad2d.numel() != n_gaussians or count.numel() != n_gaussians:
        raise RuntimeError("grad2d and count must hold one value per Gaussian")
    if gaussian_ids is not None and gaussian_ids.numel() != n_rows:
        raise RuntimeError("gaussian_ids must hold one id per row")
    if gaussian_ids is None and (radii is None or radii.numel() != 2 * n_rows):
        raise RuntimeError("dense rows need radii of the same shape as grads")
    call("gsplat_grad2d_stats", n_rows, int(n_gaussians), ptr(grads),
         ptr(gaussian_ids), ptr(radii), float(scale_x), float(scale_y),
         ptr(grad2d), ptr(count), _stream(grads))


# --------------------------------------------------------------------------
# Fused Adam  (Adam.cpp:37-66)
# --------------------------------------------------------------------------
def _adam_checks(param, param_grad, exp_avg, exp_avg_sq, valid):
    for t, n in ((param, "param"), (param_grad, "param_grad"),
                 (exp_avg, "exp_avg"), (exp_avg_sq, "exp_avg_sq")):
        check_input(t, n, _F32)
    if param_grad.shape != param.shape or exp_avg.shape != param.shape \
            or exp_avg_sq.shape != param.shape:
        raise RuntimeError("adam: param, grad and moments must have the same shape")
    if valid is not None:
        check_input(valid, "valid", torch.bool)
        if valid.dim() != 1:
            raise RuntimeError("valid should be 1D tensor")
        if valid.size(0) != param.size(0):
            raise RuntimeError("valid first dimension should match param first dimension")


def adam(
    param: Tensor,
    param_grad: Tensor,
    exp_avg: Tensor,
    exp_avg_sq: Tensor,
    valid: Optional[Tensor],
    lr: float,
    b1: float,
    b2: float,
    eps: float,
) -> None:
    _adam_checks(param, param_grad, exp_avg, exp_avg_sq, valid)
    n_rows = param.size(0) if param.dim() > 0 else 1
    row = param.numel() // n_rows if n_rows > 0 else 0
    call("gsplat_adam", ptr(param), ptr(param_grad), ptr(exp_avg),
         ptr(exp_avg_sq), ptr(valid), n_rows, row, float(lr), float(b1),
         float(b2), float(eps), _stream(param))


def adam_multi(groups, b1: float, b2: float, eps: float) -> None:
    """One launch over several tensors.

    ``groups``: iterable of (param, grad, exp_avg, exp_avg_sq, valid, lr).
    """
    entries = []
    dev = None
    for (p, g, m, v, valid, lr) in groups:
        _adam_checks(p, g, m, v, valid)
        n_rows = p.size(0) if p.dim() > 0 else 1
        row = p.numel() // n_rows if n_rows > 0 else 0
        entries.append(AdamTensor(ptr(p), ptr(g), ptr(m), ptr(v), ptr(valid),
                                  n_rows, row, float(lr)))
        dev = p
    if not entries:
        return
    arr = (AdamTensor * len(entries))(*entries)
    import ctypes
    call("gsplat_adam_multi", ctypes.cast(arr, ctypes.c_void_p), len(entries),
         float(b1), float(b2), float(eps), _stream(dev))
