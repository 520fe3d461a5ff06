"""``rasterization()``: the 3D Gaussian splatting forward pass on MI355X.

Same signature and outputs as the reference's ``gsplat.rasterization``
(gsplat/rendering.py:256-1273) for the 3DGS path: projection (dense or
packed), optional SH colour evaluation, tile intersection + sort, tile
offsets, and the tile rasterizer, all on the HIP kernels of libgsplat_hip.so.
Keyword arguments that select other model families (3DGUT ``with_ut``,
``with_eval3d``, distortion, lidar, rolling shutter, multi-GPU
``distributed``) are accepted with their defaults only and raise otherwise.
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import torch
import torch.nn.functional as F
from torch import Tensor
from typing_extensions import Literal

from .cuda import _ops
from .cuda._wrapper import (
    SUPPORTED_CHANNELS,
    CameraModel,
    Grad2dStatsSlot,
    _PackedFrontEnd,
    _PackedRowsGather,
    _PackedSphericalHarmonics,
    _project,
    _rasterize_to_pixels,
    isect_offset_encode,
    isect_tiles,
    rasterize_to_pixels,
    spherical_harmonics,
)

RenderMode = Literal["RGB", "D", "ED", "RGB+D", "RGB+ED"]
RasterizeMode = Literal["classic", "antialiased"]


def render_mode_has_color(mode: str) -> bool:
    return mode in {"RGB", "RGB+D", "RGB+ED"}


def render_mode_has_depth(mode: str) -> bool:
    return mode in {"D", "ED", "RGB+D", "RGB+ED"}


def render_mode_has_expected_depth(mode: str) -> bool:
    return mode in {"ED", "RGB+ED"}


def viewmat_to_camera_position(viewmats: Tensor) -> Tensor:
    """Camera centre -R^T t of world->camera matrices (rendering.py:216-224)."""
    R = viewmats[..., :3, :3]
    t = viewmats[..., :3, 3]
    return -(R.mT @ t.unsqueeze(-1)).squeeze(-1)


def _compute_view_dirs_packed(means, campos, batch_ids, camera_ids, gaussian_ids,
                              B: int, C: int) -> Tensor:
    """means[g] - campos[b, c] for every packed row (rendering.py:95-167)."""
    N = means.shape[-2]
    means_flat = means.reshape(B, N, 3)
    campos_flat = campos.reshape(B, C, 3)
    if B * C == 1:
        return means_flat[0, gaussian_ids] - campos_flat[0, 0]
    return means_flat[batch_ids, gaussian_ids] - campos_flat[batch_ids, camera_ids]


def compute_directions(batch_dims, means, viewmats, batch_ids=None,
                       camera_ids=None, gaussian_ids=None) -> Tensor:
    """Unit view directions (rendering.py:227-253)."""
    campos = viewmat_to_camera_position(viewmats)
    if gaussian_ids is None:
        dirs = means[..., None, :, :] - campos[..., None, :]
    else:
        B = math.prod(batch_dims)
        C = campos.shape[-2]
        dirs = _compute_view_dirs_packed(means, campos, batch_ids, camera_ids,
                                         gaussian_ids, B, C)
    return F.normalize(dirs, p=2, dim=-1)


def normalize_features_layout(features: Tensor, batch_dims: tuple, C: int,
                              trailing_dims: tuple, batch_ids=None,
                              camera_ids=None, feature_ids=None) -> Tensor:
    """Per-view or per-Gaussian features to [nnz, *] or [..., C, N, *]
    (rendering.py:170-213)."""
    B = math.prod(batch_dims)
    N = features.shape[-(len(trailing_dims) + 1)]
    if features.shape == batch_dims + (C, N) + trailing_dims:
        if feature_ids is not None:
            return features.reshape(B, C, N, *trailing_dims)[
                batch_ids, camera_ids, feature_ids]
        return features
    assert features.shape == (*batch_dims, N, *trailing_dims), features.shape
    if feature_ids is not None:
        return features.reshape(B, N, *trailing_dims)[batch_ids, feature_ids]
    return torch.broadcast_to(features.unsqueeze(len(batch_dims)),
                              batch_dims + (C, N, *trailing_dims))


def rasterization(
    means: Tensor,  # [..., N, 3]
    quats: Tensor,  # [..., N, 4]
    scales: Tensor,  # [..., N, 3]
    opacities: Tensor,  # [..., N]
    colors: Optional[Tensor],  # [..., (C,) N, D] or [..., (C,) N, K, 3]
    viewmats: Tensor,  # [..., C, 4, 4]
    Ks: Tensor,  # [..., C, 3, 3]
    width: int,
    height: int,
    near_plane: float = 0.01,
    far_plane: float = 1e10,
    radius_clip: float = 0.0,
    eps2d: float = 0.3,
    sh_degree: Optional[int] = None,
    packed: bool = True,
    tile_size: int = 16,
    backgrounds: Optional[Tensor] = None,
    render_mode: RenderMode = "RGB",
    sparse_grad: bool = False,
    absgrad: bool = False,
    rasterize_mode: RasterizeMode = "classic",
    channel_chunk: int = 32,
    distributed: bool = False,
    camera_model: CameraModel = "pinhole",
    segmented: bool = False,
    covars: Optional[Tensor] = None,
    with_ut: bool = False,
    with_eval3d: bool = False,
    return_normals: bool = False,
    global_z_order: bool = True,
    rays: Optional[Tensor] = None,
    radial_coeffs: Optional[Tensor] = None,
    tangential_coeffs: Optional[Tensor] = None,
    thin_prism_coeffs: Optional[Tensor] = None,
    ftheta_coeffs=None,
    lidar_coeffs=None,
    external_distortion_coeffs=None,
    rolling_shutter=None,
    viewmats_rs: Optional[Tensor] = None,
    ut_params=None,
    extra_signals: Optional[Tensor] = None,
    extra_signals_sh_degree: Optional[int] = None,
) -> Tuple[Tensor, Tensor, Dict]:
    """Rasterize N 3D Gaussians to a batch of I = B*C images.

    Returns ``(render_colors [..., C, H, W, X], render_alphas [..., C, H, W, 1],
    meta)`` where X is D (RGB), 1 (D/ED) or D+1 (RGB+D/RGB+ED), plus the
    channels of ``extra_signals``; ``meta`` carries the intermediate tensors
    (ids, radii, means2d, depths, conics, opacities, tiles_per_gauss,
    isect_ids, flatten_ids, isect_offsets, ...) as in the reference.
    """
    unsupported = {
        "with_ut": with_ut, "with_eval3d": with_eval3d,
        "return_normals": return_normals, "distributed": distributed,
        "rays": rays is not None, "radial_coeffs": radial_coeffs is not None,
        "tangential_coeffs": tangential_coeffs is not None,
        "thin_prism_coeffs": thin_prism_coeffs is not None,
        "ftheta_coeffs": ftheta_coeffs is not None,
        "lidar_coeffs": lidar_coeffs is not None,
        "external_distortion_coeffs": external_distortion_coeffs is not None,
        "viewmats_rs": viewmats_rs is not None, "ut_params": ut_params is not None,
        "global_z_order=False": not global_z_order,
    }
    bad = [k for k, v in unsupported.items() if v]
    if bad:
        raise NotImplementedError(
            f"rasterization(): {', '.join(bad)} not supported by the MI355X 3DGS path")
    if rolling_shutter is not None and int(rolling_shutter) != 0:
        raise NotImplementedError("rasterization(): rolling shutter not supported")
    if render_mode not in ("RGB", "D", "ED", "RGB+D", "RGB+ED"):
        raise ValueError(f"Unsupported render_mode {render_mode!r} for the 3DGS path")
    if rasterize_mode not in ("classic", "antialiased"):
        raise ValueError(f"Unsupported rasterize_mode {rasterize_mode!r}")

    meta: Dict = {}
    has_color = render_mode_has_color(render_mode)
    if has_color and colors is None:
        raise ValueError(f"colors must be provided when render_mode='{render_mode}' includes RGB.")
    if colors is None and sh_degree is not None:
        raise ValueError(f"sh_degree must be None when colors is None, got sh_degree={sh_degree}.")

    batch_dims = means.shape[:-2]
    num_batch_dims = len(batch_dims)
    B = math.prod(batch_dims)
    N = means.shape[-2]
    C = viewmats.shape[-3]
    D = colors.shape[-1] if has_color else 0
    I = B * C
    assert means.shape == batch_dims + (N, 3), means.shape
    if covars is None:
        assert quats.shape == batch_dims + (N, 4), quats.shape
        assert scales.shape == batch_dims + (N, 3), scales.shape
    else:
        assert covars.shape == batch_dims + (N, 3, 3), covars.shape
        quats, scales = None, None
        tri = ([0, 0, 0, 1, 1, 2], [0, 1, 2, 1, 2, 2])
        covars = covars[..., tri[0], tri[1]]
    assert opacities.shape == batch_dims + (N,), opacities.shape
    assert viewmats.shape == batch_dims + (C, 4, 4), viewmats.shape
    assert Ks.shape == batch_dims + (C, 3, 3), Ks.shape

    def check_features(features: Tensor, degree: Optional[int], name: str):
        channels = features.shape[-1]
        if degree is None:
            assert (features.dim() == num_batch_dims + 2
                    and features.shape[:-1] == (*batch_dims, N)) or (
                features.dim() == num_batch_dims + 3
                and features.shape[:-1] == (*batch_dims, C, N)), (
                f"{name}'s shape {features.shape} is invalid")
        else:
            assert (features.dim() == num_batch_dims + 3
                    and features.shape[:-2] == batch_dims + (N,)
                    and channels == 3) or (
                features.dim() == num_batch_dims + 4
                and features.shape[:-2] == batch_dims + (C, N)
                and channels == 3), f"{name}'s shape {features.shape} is invalid"
            assert (degree + 1) ** 2 <= features.shape[-2], features.shape

    if has_color:
        check_features(colors, sh_degree, "colors")
    if extra_signals is not None:
        check_features(extra_signals, extra_signals_sh_degree, "extra signals")

    colors_sh_degree = sh_degree if has_color else None
    proj_features = None
    per_gaussian_colors = has_color and (
        colors.shape[:num_batch_dims + 1] == batch_dims + (N,)
        and colors.dim() == num_batch_dims + (2 if colors_sh_degree is None else 3))
    fused_packed = (packed and extra_signals is None and has_color
                    and per_gaussian_colors and not viewmats.requires_grad)
    # projection, row opacities and row colours in one node (sparse_grad
    # keeps the reference's separate projection with its sparse gradients)
    front_end = fused_packed and not sparse_grad
    tile_width = math.ceil(width / float(tile_size))
    tile_height = math.ceil(height / float(tile_size))
    # the sorted tile intersection is started inside the front end when the
    # row opacities are final (no compensation factor)
    isect_req = ({"tile_size": tile_size, "tile_width": tile_width,
                  "tile_height": tile_height}
                 if front_end and rasterize_mode != "antialiased" else None)
    row_of = None
    if front_end:
        # densification statistics can join the projection backward (one
        # batch; gsplat_amd.strategy.stats.fuse_grad2d_stats)
        stats_slot = Grad2dStatsSlot(width, height, C) if B == 1 else None
        (batch_ids, camera_ids, gaussian_ids, indptr, radii, means2d, depths,
         conics, compensations, row_of, opacities, proj_features) = _PackedFrontEnd.apply(
            means.contiguous(), None if covars is None else covars.contiguous(),
            None if quats is None else quats.contiguous(),
            None if scales is None else scales.contiguous(),
            opacities.contiguous(), colors.contiguous(), viewmats.contiguous(),
            Ks.contiguous(), width, height, eps2d, near_plane, far_plane,
            radius_clip, rasterize_mode == "antialiased", camera_model,
            colors_sh_degree, isect_req, stats_slot)
        if stats_slot is not None:
            stats_slot.means2d = means2d
            meta["grad2d_stats_slot"] = stats_slot
        nnz = means2d.shape[0]
        # the rows' image ids are formed below, only if the intersection
        # was not started inside the front end (two int64 passes over the
        # rows at several cameras)
        image_ids = None
    elif packed:
        proj_results = _project(
            means, covars, quats, scales, viewmats, Ks, width, height, eps2d,
            near_plane, far_plane, radius_clip, packed, sparse_grad,
            rasterize_mode == "antialiased", camera_model, opacities,
        )
        (batch_ids, camera_ids, gaussian_ids, indptr, radii, means2d, depths,
         conics, compensations, row_of) = proj_results
        nnz = means2d.shape[0]
        # per-Gaussian -> packed rows through the inverse map (a gather whose
        # backward is a per-Gaussian sum, not an index_put)
        opacities = _PackedRowsGather.apply(
            opacities.reshape(B, N, 1), row_of, C, nnz).reshape(nnz)
        # with one image every row's image id is 0 (= camera_ids)
        image_ids = camera_ids if B * C == 1 else batch_ids * C + camera_ids
    else:
        radii, means2d, depths, conics, compensations = _project(
            means, covars, quats, scales, viewmats, Ks, width, height, eps2d,
            near_plane, far_plane, radius_clip, packed, sparse_grad,
            rasterize_mode == "antialiased", camera_model, opacities,
        )
        opacities = torch.broadcast_to(opacities[..., None, :], batch_dims + (C, N))
        batch_ids = camera_ids = gaussian_ids = indptr = None
        image_ids = None
    if compensations is not None:
        opacities = opacities * compensations
    meta.update({
        "batch_ids": batch_ids, "camera_ids": camera_ids,
        "gaussian_ids": gaussian_ids, "radii": radii, "means2d": means2d,
        "depths": depths, "conics": conics, "opacities": opacities,
    })

    if front_end:
        pass  # row colours came with the projection
    elif fused_packed:
        # packed rows with per-Gaussian colours: gather (or SH-evaluate) per
        # Gaussian through row_of instead of indexing [nnz, ...] copies
        if colors_sh_degree is None:
            proj_features = _PackedRowsGather.apply(
                colors.reshape(B, N, D), row_of, C, nnz)
        else:
            K = colors.shape[-2]
            proj_features = _PackedSphericalHarmonics.apply(
                colors_sh_degree, means.reshape(B, N, 3), colors.reshape(B, N, K, 3),
                viewmats.reshape(B, C, 4, 4).detach(), row_of, nnz)
    elif (not packed and colors_sh_degree is not None and extra_signals is None
          and per_gaussian_colors and not viewmats.requires_grad):
        # unpacked, per-Gaussian SH coefficients: the packed-row SH op over a
        # dense row map (entry (b, c, g) is row (b*C + c)*N + g where its
        # radii are positive, else -1), so the directions, the mask, the
        # +0.5 clamp and their backward stay in its two launches
        # (rendering.py:227-253, 845-873 run them as torch ops).  The
        # projection gives both radii positive or both zero; entries the
        # mask drops hold 0.5, the reference's clamp of a masked zero.
        K = colors.shape[-2]
        idx = torch.arange(B * C * N, device=means.device,
                           dtype=torch.int32).view(B, C, N)
        dense_rows = torch.where(radii.reshape(B, C, N, 2)[..., 0] > 0, idx, -1)
        proj_features = _PackedSphericalHarmonics.apply(
            colors_sh_degree, means.reshape(B, N, 3), colors.reshape(B, N, K, 3),
            viewmats.reshape(B, C, 4, 4).detach(), dense_rows, B * C * N,
            0.5).reshape(batch_dims + (C, N, 3))
    elif colors_sh_degree is None and extra_signals_sh_degree is None:
        feature_list = []
        if has_color:
            feature_list.append(colors)
        if extra_signals is not None:
            feature_list.append(extra_signals)
        if feature_list:
            proj_features = (torch.cat(feature_list, dim=-1)
                             if len(feature_list) > 1 else feature_list[0])
            proj_features = normalize_features_layout(
                proj_features, batch_dims, C, proj_features.shape[-1:],
                batch_ids, camera_ids, gaussian_ids)
    else:
        dirs = compute_directions(batch_dims, means, viewmats, batch_ids,
                                  camera_ids, gaussian_ids)
        feature_list = []
        if has_color:
            tail = colors.shape[-2:] if colors_sh_degree is not None else colors.shape[-1:]
            colors = normalize_features_layout(colors, batch_dims, C, tail,
                                               batch_ids, camera_ids, gaussian_ids)
            if colors_sh_degree is not None:
                colors = spherical_harmonics(colors_sh_degree, dirs, colors,
                                             masks=(radii > 0).all(dim=-1))
                colors = torch.clamp_min(colors + 0.5, 0.0)
            feature_list.append(colors)
        if extra_signals is not None:
            tail = (extra_signals.shape[-2:] if extra_signals_sh_degree is not None
                    else extra_signals.shape[-1:])
            es = normalize_features_layout(extra_signals, batch_dims, C, tail,
                                           batch_ids, camera_ids, gaussian_ids)
            if extra_signals_sh_degree is not None:
                es = spherical_harmonics(extra_signals_sh_degree, dirs, es,
                                         masks=(radii > 0).all(dim=-1)) + 0.5
            feature_list.append(es)
        if feature_list:
            proj_features = (torch.cat(feature_list, dim=-1)
                             if len(feature_list) > 1 else feature_list[0])

    # The depth channel, when the rasterizer reads it from the depths where
    # they lie (one call of at most 33 channels, no extra signals) instead of
    # from a copy of the features with the depths concatenated
    # (rendering.py:1025-1045 concatenates).
    depth_last = None
    if render_mode_has_depth(render_mode):
        depth_channel = depths[..., None]
        if proj_features is not None:
            if (extra_signals is None and proj_features.shape[-1] + 1
                    <= min(channel_chunk, SUPPORTED_CHANNELS[-1])):
                depth_last = depths
            else:
                proj_features = torch.cat((proj_features, depth_channel), dim=-1)
            if backgrounds is not None:
                backgrounds = torch.cat(
                    [backgrounds,
                     torch.zeros((*batch_dims, C, 1), device=backgrounds.device)],
                    dim=-1)
        else:
            proj_features = depth_channel
            if backgrounds is not None:
                backgrounds = torch.zeros((*batch_dims, C, 1), device=backgrounds.device)
    assert proj_features is not None

    if isect_req is not None and "state" in isect_req:
        # the tile-first sorted intersection also gives the tile offsets
        tiles_per_gauss, isect_ids, flatten_ids, isect_offsets = _ops.isect_emit_sorted(
            isect_req.pop("state"))
    else:
        if front_end:
            image_ids = camera_ids if B * C == 1 else batch_ids * C + camera_ids
        tiles_per_gauss, isect_ids, flatten_ids = isect_tiles(
            means2d, radii, depths, tile_size, tile_width, tile_height,
            segmented=segmented, packed=packed, n_images=I, image_ids=image_ids,
            gaussian_ids=gaussian_ids, conics=conics, opacities=opacities,
        )
        isect_offsets = isect_offset_encode(isect_ids, I, tile_width, tile_height)
    isect_offsets = isect_offsets.reshape(batch_dims + (C, tile_height, tile_width))
    meta.update({
        "tile_width": tile_width, "tile_height": tile_height,
        "tiles_per_gauss": tiles_per_gauss, "isect_ids": isect_ids,
        "flatten_ids": flatten_ids, "isect_offsets": isect_offsets,
        "width": width, "height": height, "tile_size": tile_size,
        "n_batches": B, "n_cameras": C,
    })

    # the expected depth divided by the alpha inside the rasterizer
    # (rendering.py:1259-1267 forms it with torch ops on the render)
    n_feat = proj_features.shape[-1] + (1 if depth_last is not None else 0)
    ed_in_kernel = (render_mode_has_expected_depth(render_mode) and extra_signals is None
                    and n_feat <= min(channel_chunk, SUPPORTED_CHANNELS[-1]))
    if ed_in_kernel or depth_last is not None:
        render_colors, render_alphas = _rasterize_to_pixels(
            means2d, conics, proj_features, opacities, width, height, tile_size,
            isect_offsets, flatten_ids, backgrounds=backgrounds, packed=packed,
            absgrad=absgrad, expected_depth_channel=n_feat - 1 if ed_in_kernel else -1,
            color_last=depth_last)
    elif proj_features.shape[-1] > channel_chunk:
        n_chunks = (proj_features.shape[-1] + channel_chunk - 1) // channel_chunk
        render_colors, render_alphas = [], []
        for i in range(n_chunks):
            sl = slice(i * channel_chunk, (i + 1) * channel_chunk)
            rc, ra = rasterize_to_pixels(
                means2d, conics, proj_features[..., sl], opacities, width, height,
                tile_size, isect_offsets, flatten_ids,
                backgrounds=backgrounds[..., sl] if backgrounds is not None else None,
                packed=packed, absgrad=absgrad)
            render_colors.append(rc)
            render_alphas.append(ra)
        render_colors = torch.cat(render_colors, dim=-1)
        render_alphas = render_alphas[0]
    else:
        render_colors, render_alphas = rasterize_to_pixels(
            means2d, conics, proj_features, opacities, width, height, tile_size,
            isect_offsets, flatten_ids, backgrounds=backgrounds, packed=packed,
            absgrad=absgrad)

    if extra_signals is not None:
        E = extra_signals.shape[-1]
        meta["render_extra_signals"] = render_colors[..., D:D + E]
        if render_mode_has_depth(render_mode):
            render_depth = render_colors[..., -1:]
            if render_mode_has_expected_depth(render_mode):
                render_depth = render_depth / render_alphas.clamp(min=1e-10)
            render_colors = torch.cat([render_colors[..., 0:D], render_depth], dim=-1)
        else:
            render_colors = render_colors[..., 0:D]
    elif render_mode_has_expected_depth(render_mode) and not ed_in_kernel:
        render_colors = torch.cat(
            [render_colors[..., :-1],
             render_colors[..., -1:] / render_alphas.clamp(min=1e-10)], dim=-1)
    return render_colors, render_alphas, meta
