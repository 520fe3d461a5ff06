"""Python API of the splatting ops, argument-for-argument the reference's
``gsplat.cuda._wrapper`` for the 3DGS hot path (gsplat/cuda/_wrapper.py):

    fully_fused_projection  (:479-631)   spherical_harmonics (:342-372)
    isect_tiles             (:635-730)   isect_offset_encode (:807-826)
    rasterize_to_pixels     (:829-961)   adam                (:326-339)

with the autograd Functions _FullyFusedProjection (:1464-1594),
_FullyFusedProjectionPacked (:2107-2326), _SphericalHarmonics (:2329-2363)
and _RasterizeToPixels (:1709-1836).  The kernels behind them are the HIP
kernels of libgsplat_hip.so, reached through ``_ops``.
"""

from __future__ import annotations

import math
import weakref
from typing import Callable, Optional, Tuple

import torch
from torch import Tensor
from typing_extensions import Literal

from . import _ops
from ._backend import CameraModelType, _C  # noqa: F401  (registers torch.ops.gsplat)

CameraModel = Literal["pinhole", "ortho", "fisheye", "ftheta", "lidar"]

# Channel counts with a compiled rasterizer instantiation.
SUPPORTED_CHANNELS = (1, 2, 3, 4, 5, 8, 9, 16, 17, 32, 33)
CHANNEL_CHUNK = 32


def _make_lazy_cuda_func(name: str) -> Callable:
    """Direct handle to the op implementation (same arguments as
    ``torch.ops.gsplat.<name>``, without the dispatcher round trip)."""
    return getattr(_ops, name)


def _make_lazy_cuda_obj(name: str):
    obj = _C
    for part in name.split("."):
        obj = getattr(obj, part)
    return obj


def _camera_model_type(camera_model: str) -> int:
    if camera_model not in ("pinhole", "ortho"):
        raise NotImplementedError(
            f"camera_model={camera_model!r}: only 'pinhole' and 'ortho' are "
            "implemented by the MI355X kernels")
    return int(_make_lazy_cuda_obj(f"CameraModelType.{camera_model.upper()}"))


def has_3dgs() -> bool:
    # the reference's probe (_wrapper.py:181-184)
    return hasattr(torch.ops.gsplat, "projection_ewa_simple_fwd")


def has_adam() -> bool:
    return hasattr(torch.ops.gsplat, "adam")


def has_2dgs() -> bool:
    return False


def has_3dgut() -> bool:
    return False


def has_reloc() -> bool:
    return False


def has_camera_wrappers() -> bool:
    return False


def adam(
    param: Tensor,
    param_grad: Tensor,
    exp_avg: Tensor,
    exp_avg_sq: Tensor,
    valid: Tensor,
    lr: float,
    b1: float,
    b2: float,
    eps: float,
) -> None:
    _make_lazy_cuda_func("adam")(
        param, param_grad, exp_avg, exp_avg_sq, valid, lr, b1, b2, eps
    )


def spherical_harmonics(
    degrees_to_use: int,
    dirs: Tensor,  # [..., 3]
    coeffs: Tensor,  # [..., K, 3]
    masks: Optional[Tensor] = None,  # [...,]
) -> Tensor:
    """Computes spherical harmonics colours. [..., 3]"""
    assert (degrees_to_use + 1) ** 2 <= coeffs.shape[-2], coeffs.shape
    batch_dims = dirs.shape[:-1]
    assert dirs.shape == batch_dims + (3,), dirs.shape
    assert (
        (len(coeffs.shape) == len(batch_dims) + 2)
        and coeffs.shape[:-2] == batch_dims
        and coeffs.shape[-1] == 3
    ), coeffs.shape
    if masks is not None:
        assert masks.shape == batch_dims, masks.shape
        masks = masks.contiguous()
    return _SphericalHarmonics.apply(
        degrees_to_use, dirs.contiguous(), coeffs.contiguous(), masks
    )


def proj(
    means: Tensor,  # [..., C, N, 3]
    covars: Tensor,  # [..., C, N, 3, 3]
    Ks: Tensor,  # [..., C, 3, 3]
    width: int,
    height: int,
    camera_model: CameraModel = "pinhole",
) -> Tuple[Tensor, Tensor]:
    """Projection of camera-space Gaussians (perspective or orthographic):
    (means2d [..., C, N, 2], covars2d [..., C, N, 2, 2])."""
    assert (
        camera_model != "ftheta"
    ), "ftheta camera is only supported via UT, please set with_ut=True in the rasterization()"
    batch_dims = means.shape[:-3]
    C, N = means.shape[-3:-1]
    assert means.shape == batch_dims + (C, N, 3), means.shape
    assert covars.shape == batch_dims + (C, N, 3, 3), covars.shape
    assert Ks.shape == batch_dims + (C, 3, 3), Ks.shape
    return _Proj.apply(means.contiguous(), covars.contiguous(), Ks.contiguous(), width,
                       height, camera_model)


def fully_fused_projection(
    means: Tensor,  # [..., N, 3]
    covars: Optional[Tensor],  # [..., N, 6] or None
    quats: Optional[Tensor],  # [..., N, 4] or None
    scales: Optional[Tensor],  # [..., N, 3] or None
    viewmats: Tensor,  # [..., C, 4, 4]
    Ks: Tensor,  # [..., C, 3, 3]
    width: int,
    height: int,
    eps2d: float = 0.3,
    near_plane: float = 0.01,
    far_plane: float = 1e10,
    radius_clip: float = 0.0,
    packed: bool = False,
    sparse_grad: bool = False,
    calc_compensations: bool = False,
    camera_model: CameraModel = "pinhole",
    opacities: Optional[Tensor] = None,  # [..., N] or None
) -> Tuple[Tensor, ...]:
    """Projects Gaussians to 2D (EWA splatting).

    Returns, if ``packed``: (batch_ids, camera_ids, gaussian_ids, indptr, radii,
    means2d, depths, conics, compensations) over the nnz visible rows; else
    (radii, means2d, depths, conics, compensations) of shape [..., C, N, *].
    """
    out = _project(means, covars, quats, scales, viewmats, Ks, width, height,
                   eps2d, near_plane, far_plane, radius_clip, packed, sparse_grad,
                   calc_compensations, camera_model, opacities)
    return out[:9] if packed else out


def _project(means, covars, quats, scales, viewmats, Ks, width, height, eps2d,
             near_plane, far_plane, radius_clip, packed, sparse_grad,
             calc_compensations, camera_model, opacities):
    """fully_fused_projection; the packed form also returns ``row_of``."""
    batch_dims = means.shape[:-2]
    N = means.shape[-2]
    C = viewmats.shape[-3]
    assert means.shape == batch_dims + (N, 3), means.shape
    assert viewmats.shape == batch_dims + (C, 4, 4), viewmats.shape
    assert Ks.shape == batch_dims + (C, 3, 3), Ks.shape
    means = means.contiguous()
    if covars is not None:
        assert covars.shape == batch_dims + (N, 6), covars.shape
        covars = covars.contiguous()
    else:
        assert quats is not None, "covars or quats is required"
        assert scales is not None, "covars or scales is required"
        assert quats.shape == batch_dims + (N, 4), quats.shape
        assert scales.shape == batch_dims + (N, 3), scales.shape
        quats = quats.contiguous()
        scales = scales.contiguous()
    if sparse_grad:
        assert packed, "sparse_grad is only supported when packed is True"
        assert batch_dims == (), "sparse_grad does not support batch dimensions"
    if opacities is not None:
        assert opacities.shape == batch_dims + (N,), opacities.shape
        opacities = opacities.contiguous()
    viewmats = viewmats.contiguous()
    Ks = Ks.contiguous()
    if packed:
        return _FullyFusedProjectionPacked.apply(
            means, covars, quats, scales, viewmats, Ks, width, height, eps2d,
            near_plane, far_plane, radius_clip, sparse_grad, calc_compensations,
            camera_model, opacities,
        )
    return _FullyFusedProjection.apply(
        means, covars, quats, scales, viewmats, Ks, width, height, eps2d,
        near_plane, far_plane, radius_clip, calc_compensations, camera_model,
        opacities,
    )


@torch.no_grad()
def isect_tiles(
    means2d: Tensor,  # [..., N, 2] or [nnz, 2]
    radii: Tensor,  # [..., N, 2] or [nnz, 2]
    depths: Tensor,  # [..., N] or [nnz]
    tile_size: int,
    tile_width: int,
    tile_height: int,
    sort: bool = True,
    segmented: bool = False,
    packed: bool = False,
    n_images: Optional[int] = None,
    image_ids: Optional[Tensor] = None,
    gaussian_ids: Optional[Tensor] = None,
    conics: Optional[Tensor] = None,  # enables the ellipse test with opacities
    opacities: Optional[Tensor] = None,
) -> Tuple[Tensor, Tensor, Tensor]:
    """Maps projected Gaussians to intersecting tiles.

    Returns (tiles_per_gauss int32, isect_ids int64 image|tile|depth-bits,
    flatten_ids int32 index into [I * N] or [nnz]).
    """
    if packed:
        nnz = means2d.size(0)
        assert means2d.shape == (nnz, 2), means2d.shape
        assert radii.shape == (nnz, 2), radii.shape
        assert depths.shape == (nnz,), depths.shape
        if conics is not None:
            assert conics.shape == (nnz, 3), conics.shape
        if opacities is not None:
            assert opacities.shape == (nnz,), opacities.shape
        assert image_ids is not None, "image_ids is required if packed is True"
        assert gaussian_ids is not None, "gaussian_ids is required if packed is True"
        assert n_images is not None, "n_images is required if packed is True"
        image_ids = image_ids.contiguous()
        gaussian_ids = gaussian_ids.contiguous()
        I = n_images
    else:
        image_dims = means2d.shape[:-2]
        I = math.prod(image_dims)
        N = means2d.shape[-2]
        assert means2d.shape == image_dims + (N, 2), means2d.shape
        assert radii.shape == image_dims + (N, 2), radii.shape
        assert depths.shape == image_dims + (N,), depths.shape
        if conics is not None:
            assert conics.shape == image_dims + (N, 3), conics.shape
        if opacities is not None:
            assert opacities.shape == image_dims + (N,), opacities.shape
    return _make_lazy_cuda_func("intersect_tile")(
        means2d.contiguous(),
        radii.contiguous(),
        depths.contiguous(),
        conics.contiguous() if conics is not None else None,
        opacities.contiguous() if opacities is not None else None,
        image_ids,
        gaussian_ids,
        I,
        tile_size,
        tile_width,
        tile_height,
        sort,
        segmented,
    )


@torch.no_grad()
def isect_offset_encode(
    isect_ids: Tensor, n_images: int, tile_width: int, tile_height: int
) -> Tensor:
    """Encodes intersection ids to tile start offsets. [I, tile_height, tile_width]"""
    return _make_lazy_cuda_func("intersect_offset")(
        isect_ids.contiguous(), n_images, tile_width, tile_height
    )


def _pad_channels(channels: int) -> int:
    for c in SUPPORTED_CHANNELS:
        if c >= channels:
            return c
    raise ValueError(f"Unsupported number of color channels: {channels}")


def rasterize_to_pixels(
    means2d: Tensor,  # [..., N, 2] or [nnz, 2]
    conics: Tensor,  # [..., N, 3] or [nnz, 3]
    colors: Tensor,  # [..., N, channels] or [nnz, channels]
    opacities: Tensor,  # [..., N] or [nnz]
    image_width: int,
    image_height: int,
    tile_size: int,
    isect_offsets: Tensor,  # [..., tile_height, tile_width]
    flatten_ids: Tensor,  # [n_isects]
    backgrounds: Optional[Tensor] = None,  # [..., channels]
    masks: Optional[Tensor] = None,  # [..., tile_height, tile_width]
    packed: bool = False,
    absgrad: bool = False,
) -> Tuple[Tensor, Tensor]:
    """Rasterizes Gaussians to pixels.

    Returns (render_colors [..., H, W, channels], render_alphas [..., H, W, 1]).
    Channel counts without a compiled kernel are zero-padded to the next one;
    more than 33 channels are rendered in 32-channel chunks (for absgrad, the
    chunks' |dL/dmean2d| are summed).
    """
    return _rasterize_to_pixels(
        means2d, conics, colors, opacities, image_width, image_height, tile_size,
        isect_offsets, flatten_ids, backgrounds, masks, packed, absgrad)


def _rasterize_to_pixels(
    means2d: Tensor,
    conics: Tensor,
    colors: Tensor,
    opacities: Tensor,
    image_width: int,
    image_height: int,
    tile_size: int,
    isect_offsets: Tensor,
    flatten_ids: Tensor,
    backgrounds: Optional[Tensor] = None,
    masks: Optional[Tensor] = None,
    packed: bool = False,
    absgrad: bool = False,
    expected_depth_channel: int = -1,
    color_last: Optional[Tensor] = None,
) -> Tuple[Tensor, Tensor]:
    """rasterize_to_pixels; with ``expected_depth_channel`` >= 0 (at most 33
    channels) that channel of the render comes out divided by
    max(alpha, 1e-10), the expected depth rasterization() forms for render
    modes ED and RGB+ED (rendering.py:1259-1267), inside the rasterizer
    kernels instead of by torch ops on the render and their backward.  With
    ``color_last`` (one value per row: [nnz] packed, [..., N] otherwise) the
    render has a last channel more, taken from it: rasterization()'s depth
    channel (rendering.py:1025-1045), which the replay kernels read where it
    lies instead of from a concatenated copy of the colours."""
    image_dims = means2d.shape[:-2]
    channels = colors.shape[-1]
    device = means2d.device
    if color_last is not None:
        assert color_last.shape == colors.shape[:-1], color_last.shape
        if channels + 1 > SUPPORTED_CHANNELS[-1] or \
                _pad_channels(channels + 1) != channels + 1:
            # a padded or chunked render takes the concatenated colours
            colors = torch.cat([colors, color_last[..., None]], dim=-1)
            color_last = None
        channels = colors.shape[-1] + (1 if color_last is not None else 0)
    if packed:
        nnz = means2d.size(0)
        assert means2d.shape == (nnz, 2), means2d.shape
        assert conics.shape == (nnz, 3), conics.shape
        assert colors.shape[0] == nnz, colors.shape
        assert opacities.shape == (nnz,), opacities.shape
    else:
        N = means2d.size(-2)
        assert means2d.shape == image_dims + (N, 2), means2d.shape
        assert conics.shape == image_dims + (N, 3), conics.shape
        assert colors.shape == image_dims + (N, colors.shape[-1]), colors.shape
        assert opacities.shape == image_dims + (N,), opacities.shape
    if backgrounds is not None:
        # one background per image: packed rows carry no image dims, so the
        # images are those of the tile grid (the reference checks packed
        # backgrounds against the rows' empty dims, _wrapper.py:884-886,
        # which no [..., C, channels] background passes)
        bg_dims = tuple(isect_offsets.shape[:-2]) if packed else image_dims
        assert backgrounds.shape == bg_dims + (channels,), backgrounds.shape
        backgrounds = backgrounds.contiguous()
    if masks is not None:
        assert masks.shape == isect_offsets.shape, masks.shape
        masks = masks.contiguous()
    if channels > 513 or channels == 0:
        raise ValueError(f"Unsupported number of color channels: {channels}")

    tile_height, tile_width = isect_offsets.shape[-2:]
    assert (
        tile_height * tile_size >= image_height
    ), f"Assert Failed: {tile_height} * {tile_size} >= {image_height}"
    assert (
        tile_width * tile_size >= image_width
    ), f"Assert Failed: {tile_width} * {tile_size} >= {image_width}"

    means2d = means2d.contiguous()
    conics = conics.contiguous()
    opacities = opacities.contiguous()
    isect_offsets = isect_offsets.contiguous()
    flatten_ids = flatten_ids.contiguous()

    if color_last is not None:
        # no padding: the channel count is a compiled one
        return _RasterizeToPixels.apply(
            means2d, conics, colors.contiguous(), opacities, backgrounds, masks,
            image_width, image_height, tile_size, isect_offsets, flatten_ids,
            absgrad, expected_depth_channel, color_last.contiguous())

    def one(cols: Tensor, bgs: Optional[Tensor]) -> Tuple[Tensor, Tensor]:
        c = cols.shape[-1]
        pc = _pad_channels(c)
        if pc != c:
            cols = torch.cat(
                [cols, torch.zeros(*cols.shape[:-1], pc - c, device=device)], dim=-1)
            if bgs is not None:
                bgs = torch.cat(
                    [bgs, torch.zeros(*bgs.shape[:-1], pc - c, device=device)], dim=-1)
        rc, ra = _RasterizeToPixels.apply(
            means2d, conics, cols.contiguous(), opacities, bgs, masks,
            image_width, image_height, tile_size, isect_offsets, flatten_ids,
            absgrad, expected_depth_channel, None,
        )
        if pc != c:
            rc = rc[..., :c]
        return rc, ra

    if channels <= SUPPORTED_CHANNELS[-1]:
        return one(colors, backgrounds)
    if expected_depth_channel >= 0:
        raise ValueError("the in-kernel expected depth takes at most "
                         f"{SUPPORTED_CHANNELS[-1]} channels")
    outs, alphas = [], None
    for s in range(0, channels, CHANNEL_CHUNK):
        rc, ra = one(
            colors[..., s:s + CHANNEL_CHUNK],
            backgrounds[..., s:s + CHANNEL_CHUNK] if backgrounds is not None else None,
        )
        outs.append(rc)
        if alphas is None:
            alphas = ra
    return torch.cat(outs, dim=-1), alphas


def quat_scale_to_covar_preci(
    quats: Tensor,
    scales: Tensor,
    compute_covar: bool = True,
    compute_preci: bool = True,
    triu: bool = False,
) -> Tuple[Optional[Tensor], Optional[Tensor]]:
    """Covariance R S^2 R^T and precision R S^-2 R^T matrices from (unnormalized)
    quaternions [..., 4] and scales [..., 3]; [..., 6] upper triangles when
    ``triu``, else [..., 3, 3].  Signature of gsplat/cuda/_wrapper.py:375-414."""
    batch_dims = quats.shape[:-1]
    assert quats.shape == batch_dims + (4,), quats.shape
    assert scales.shape == batch_dims + (3,), scales.shape
    covars, precis = _QuatScaleToCovarPreci.apply(
        quats.contiguous(), scales.contiguous(), compute_covar, compute_preci, triu)
    return covars if compute_covar else None, precis if compute_preci else None


class _QuatScaleToCovarPreci(torch.autograd.Function):
    """gsplat/cuda/_wrapper.py:1355-1400."""

    @staticmethod
    def forward(ctx, quats, scales, compute_covar, compute_preci, triu):
        covars, precis = _make_lazy_cuda_func("quat_scale_to_covar_preci_fwd")(
            quats, scales, compute_covar, compute_preci, triu)
        ctx.save_for_backward(quats, scales)
        ctx.compute_covar = compute_covar
        ctx.compute_preci = compute_preci
        ctx.triu = triu
        return covars, precis

    @staticmethod
    def backward(ctx, v_covars, v_precis):
        quats, scales = ctx.saved_tensors
        if ctx.compute_covar and v_covars is not None and v_covars.is_sparse:
            v_covars = v_covars.to_dense()
        if ctx.compute_preci and v_precis is not None and v_precis.is_sparse:
            v_precis = v_precis.to_dense()
        v_quats, v_scales = _make_lazy_cuda_func("quat_scale_to_covar_preci_bwd")(
            quats, scales, ctx.triu,
            v_covars.contiguous() if ctx.compute_covar and v_covars is not None else None,
            v_precis.contiguous() if ctx.compute_preci and v_precis is not None else None)
        return v_quats, v_scales, None, None, None


def rasterize_to_indices_in_range(
    range_start: int,
    range_end: int,
    transmittances: Tensor,
    means2d: Tensor,
    conics: Tensor,
    opacities: Tensor,
    image_width: int,
    image_height: int,
    tile_size: int,
    isect_offsets: Tensor,
    flatten_ids: Tensor,
) -> Tuple[Tensor, Tensor, Tensor]:
    """The (Gaussian id, pixel id, image id) of every pixel-Gaussian pair
    composited over the isect batches [range_start, range_end) from the given
    transmittances [..., H, W]; means2d [..., N, 2].  Signature and results of
    gsplat/cuda/_wrapper.py:1274-1352."""
    image_dims = means2d.shape[:-2]
    tile_height, tile_width = isect_offsets.shape[-2:]
    N = means2d.shape[-2]
    assert transmittances.shape == image_dims + (image_height, image_width), \
        transmittances.shape
    assert means2d.shape == image_dims + (N, 2), means2d.shape
    assert conics.shape == image_dims + (N, 3), conics.shape
    assert opacities.shape == image_dims + (N,), opacities.shape
    assert isect_offsets.shape == image_dims + (tile_height, tile_width), \
        isect_offsets.shape
    assert tile_height * tile_size >= image_height
    assert tile_width * tile_size >= image_width
    out_gauss_ids, out_indices = _make_lazy_cuda_func("rasterize_to_indices_3dgs")(
        range_start, range_end, transmittances.contiguous(), means2d.contiguous(),
        conics.contiguous(), opacities.contiguous(), image_width, image_height,
        tile_size, isect_offsets.contiguous(), flatten_ids.contiguous())
    out_pixel_ids = out_indices % (image_width * image_height)
    out_image_ids = out_indices // (image_width * image_height)
    return out_gauss_ids, out_pixel_ids, out_image_ids


class _Proj(torch.autograd.Function):
    """Autograd node of ``proj`` (reference _wrapper.py:1403-1460)."""

    @staticmethod
    def forward(ctx, means, covars, Ks, width, height, camera_model="pinhole"):
        camera_model_type = _camera_model_type(camera_model)
        means2d, covars2d = _make_lazy_cuda_func("projection_ewa_simple_fwd")(
            means, covars, Ks, width, height, camera_model_type)
        ctx.save_for_backward(means, covars, Ks)
        ctx.width = width
        ctx.height = height
        ctx.camera_model_type = camera_model_type
        return means2d, covars2d

    @staticmethod
    def backward(ctx, v_means2d, v_covars2d):
        means, covars, Ks = ctx.saved_tensors
        if v_means2d is None:
            v_means2d = torch.zeros(means.shape[:-1] + (2,), dtype=means.dtype,
                                    device=means.device)
        if v_covars2d is None:
            v_covars2d = torch.zeros(means.shape[:-1] + (2, 2), dtype=means.dtype,
                                     device=means.device)
        v_means, v_covars = _make_lazy_cuda_func("projection_ewa_simple_bwd")(
            means, covars, Ks, ctx.width, ctx.height, ctx.camera_model_type,
            v_means2d.contiguous(), v_covars2d.contiguous())
        return v_means, v_covars, None, None, None, None


class _FullyFusedProjection(torch.autograd.Function):
    """Projects Gaussians to 2D (dense [..., C, N] outputs)."""

    @staticmethod
    def forward(
        ctx,
        means: Tensor,
        covars: Optional[Tensor],
        quats: Optional[Tensor],
        scales: Optional[Tensor],
        viewmats: Tensor,
        Ks: Tensor,
        width: int,
        height: int,
        eps2d: float,
        near_plane: float,
        far_plane: float,
        radius_clip: float,
        calc_compensations: bool,
        camera_model: CameraModel = "pinhole",
        opacities: Optional[Tensor] = None,
    ):
        cm = _camera_model_type(camera_model)
        radii, means2d, depths, conics, compensations = _make_lazy_cuda_func(
            "projection_ewa_3dgs_fused_fwd"
        )(means, covars, quats, scales, opacities, viewmats, Ks, width, height,
          eps2d, near_plane, far_plane, radius_clip, calc_compensations, cm)
        if not calc_compensations:
            compensations = None
        ctx.save_for_backward(
            means, covars, quats, scales, viewmats, Ks, radii, conics, compensations
        )
        ctx.width = width
        ctx.height = height
        ctx.eps2d = eps2d
        ctx.camera_model_type = cm
        ctx.mark_non_differentiable(radii)
        return radii, means2d, depths, conics, compensations

    @staticmethod
    def backward(ctx, v_radii, v_means2d, v_depths, v_conics, v_compensations):
        (means, covars, quats, scales, viewmats, Ks, radii, conics,
         compensations) = ctx.saved_tensors
        if compensations is None:
            v_compensations = None
        elif v_compensations is not None:
            v_compensations = v_compensations.contiguous()
        v_means, v_covars, v_quats, v_scales, v_viewmats = _make_lazy_cuda_func(
            "projection_ewa_3dgs_fused_bwd"
        )(means, covars, quats, scales, viewmats, Ks, ctx.width, ctx.height,
          ctx.eps2d, ctx.camera_model_type, radii, conics, compensations,
          v_means2d.contiguous(), v_depths.contiguous(), v_conics.contiguous(),
          v_compensations, ctx.needs_input_grad[4])
        if not ctx.needs_input_grad[0]:
            v_means = None
        if not ctx.needs_input_grad[1]:
            v_covars = None
        if not ctx.needs_input_grad[2]:
            v_quats = None
        if not ctx.needs_input_grad[3]:
            v_scales = None
        if not ctx.needs_input_grad[4]:
            v_viewmats = None
        return (v_means, v_covars, v_quats, v_scales, v_viewmats,
                None, None, None, None, None, None, None, None, None, None)


class _FullyFusedProjectionPacked(torch.autograd.Function):
    """Projects Gaussians to 2D; returns the visible rows packed, followed by
    ``row_of`` [B*C*N] int32 (the packed row of each (b, c, g), or -1), which
    ``fully_fused_projection`` drops and ``rasterization`` uses for its
    per-Gaussian gathers."""

    @staticmethod
    def forward(
        ctx,
        means: Tensor,
        covars: Optional[Tensor],
        quats: Optional[Tensor],
        scales: Optional[Tensor],
        viewmats: Tensor,
        Ks: Tensor,
        width: int,
        height: int,
        eps2d: float,
        near_plane: float,
        far_plane: float,
        radius_clip: float,
        sparse_grad: bool,
        calc_compensations: bool,
        camera_model: CameraModel = "pinhole",
        opacities: Optional[Tensor] = None,
    ):
        cm = _camera_model_type(camera_model)
        (indptr, batch_ids, camera_ids, gaussian_ids, radii, means2d, depths,
         conics, compensations, row_of) = _ops.projection_packed_fwd_with_row_map(
            means, covars, quats, scales, opacities, viewmats, Ks, width, height,
            eps2d, near_plane, far_plane, radius_clip, calc_compensations, cm)
        if not calc_compensations:
            compensations = None
        ctx.save_for_backward(batch_ids, camera_ids, gaussian_ids, means, covars,
                              quats, scales, viewmats, Ks, conics, compensations,
                              row_of)
        # unused outputs (depths, often) reach backward as None, not zeros
        ctx.set_materialize_grads(False)
        ctx.width = width
        ctx.height = height
        ctx.eps2d = eps2d
        ctx.sparse_grad = sparse_grad
        ctx.camera_model_type = cm
        ctx.mark_non_differentiable(batch_ids, camera_ids, gaussian_ids, indptr, radii,
                                    row_of)
        return (batch_ids, camera_ids, gaussian_ids, indptr, radii, means2d,
                depths, conics, compensations, row_of)

    @staticmethod
    def backward(ctx, v_batch_ids, v_camera_ids, v_gaussian_ids, v_indptr,
                 v_radii, v_means2d, v_depths, v_conics, v_compensations, v_row_of):
        (batch_ids, camera_ids, gaussian_ids, means, covars, quats, scales,
         viewmats, Ks, conics, compensations, row_of) = ctx.saved_tensors
        sparse_grad = ctx.sparse_grad
        if compensations is None:
            v_compensations = None
        elif v_compensations is not None:
            v_compensations = v_compensations.contiguous()
        v_means2d = (torch.zeros_like(conics[:, :2]) if v_means2d is None
                     else v_means2d.contiguous())
        v_conics = torch.zeros_like(conics) if v_conics is None else v_conics.contiguous()
        if sparse_grad:
            if v_depths is None:
                v_depths = torch.zeros_like(conics[:, 0])
            v_means, v_covars, v_quats, v_scales, v_viewmats = _make_lazy_cuda_func(
                "projection_ewa_3dgs_packed_bwd"
            )(means, covars, quats, scales, viewmats, Ks, ctx.width, ctx.height,
              ctx.eps2d, ctx.camera_model_type, batch_ids, camera_ids, gaussian_ids,
              conics, compensations, v_means2d, v_depths.contiguous(),
              v_conics, v_compensations, ctx.needs_input_grad[4], sparse_grad)
        else:
            # dense gradients straight from the row map: one pass, no fill
            v_means, v_covars, v_quats, v_scales, v_viewmats = _ops.projection_packed_bwd_rows(
                means, covars, quats, scales, viewmats, Ks, ctx.width, ctx.height,
                ctx.eps2d, ctx.camera_model_type, row_of, conics, compensations,
                v_means2d, None if v_depths is None else v_depths.contiguous(),
                v_conics, v_compensations, ctx.needs_input_grad[4])
        coalesced = len(viewmats) == 1

        def sparse(values, like):
            return torch.sparse_coo_tensor(indices=gaussian_ids[None], values=values,
                                           size=like.shape, is_coalesced=coalesced)

        if not ctx.needs_input_grad[0]:
            v_means = None
        elif sparse_grad:
            v_means = sparse(v_means, means)
        if not ctx.needs_input_grad[1]:
            v_covars = None
        elif sparse_grad:
            v_covars = sparse(v_covars, covars)
        if not ctx.needs_input_grad[2]:
            v_quats = None
        elif sparse_grad:
            v_quats = sparse(v_quats, quats)
        if not ctx.needs_input_grad[3]:
            v_scales = None
        elif sparse_grad:
            v_scales = sparse(v_scales, scales)
        if not ctx.needs_input_grad[4]:
            v_viewmats = None
        return (v_means, v_covars, v_quats, v_scales, v_viewmats,
                None, None, None, None, None, None, None, None, None, None, None)


class _SphericalHarmonics(torch.autograd.Function):
    """Spherical harmonics colour evaluation."""

    @staticmethod
    def forward(ctx, sh_degree: int, dirs: Tensor, coeffs: Tensor, masks: Optional[Tensor]):
        colors = _make_lazy_cuda_func("spherical_harmonics_fwd")(
            sh_degree, dirs, coeffs, masks)
        ctx.save_for_backward(dirs, coeffs, masks)
        ctx.sh_degree = sh_degree
        return colors

    @staticmethod
    def backward(ctx, v_colors: Tensor):
        dirs, coeffs, masks = ctx.saved_tensors
        compute_v_dirs = ctx.needs_input_grad[1]
        v_coeffs, v_dirs = _make_lazy_cuda_func("spherical_harmonics_bwd")(
            ctx.sh_degree, dirs, coeffs, masks, v_colors.contiguous(), compute_v_dirs)
        if not compute_v_dirs:
            v_dirs = None
        return None, v_dirs, v_coeffs, None


class _PackedRowsGather(torch.autograd.Function):
    """out[row_of[b, c, g]] = src[b, g]: a per-Gaussian feature to its packed
    rows (the reference indexes src[batch_ids, gaussian_ids],
    rendering.py:782, 170-213).  Backward sums each Gaussian's rows, driven
    by Gaussian (no index_put)."""

    @staticmethod
    def forward(ctx, src: Tensor, row_of: Tensor, C: int, nnz: int):
        ctx.save_for_backward(row_of)
        ctx.dims = (src.shape[0], C, src.shape[1])
        return _ops.rows_gather(src.contiguous(), row_of, C, nnz)

    @staticmethod
    def backward(ctx, v_out: Tensor):
        (row_of,) = ctx.saved_tensors
        B, C, N = ctx.dims
        v_src = None
        if ctx.needs_input_grad[0]:
            v_src = _ops.rows_scatter_sum(v_out.contiguous(), row_of, B, C, N)
        return v_src, None, None, None


class _PackedSphericalHarmonics(torch.autograd.Function):
    """Clamped SH colour of every packed row, max(SH(mean - campos) + 0.5, 0)
    with campos = -R^T t taken from the view matrices in the kernel,
    evaluated per Gaussian (the reference's compute_directions + gathers +
    spherical_harmonics + clamp_min, rendering.py:227-253, 845-873).  The
    view matrices get no gradient (the caller detaches them)."""

    @staticmethod
    def forward(ctx, degree: int, means: Tensor, coeffs: Tensor, viewmats: Tensor,
                row_of: Tensor, nnz: int, fill: Optional[float] = None):
        # ``fill``: the value of rows no entry of row_of names (a dense row
        # map leaves the culled entries' rows unnamed)
        means = means.contiguous()
        coeffs = coeffs.contiguous()
        viewmats = viewmats.contiguous()
        colors = _ops.sh_rows_fwd(degree, means, viewmats, coeffs, row_of, nnz,
                                  fill=fill)
        ctx.save_for_backward(means, coeffs, viewmats, row_of)
        ctx.degree = degree
        return colors

    @staticmethod
    def backward(ctx, v_colors: Tensor):
        means, coeffs, viewmats, row_of = ctx.saved_tensors
        v_coeffs, v_means = _ops.sh_rows_bwd(ctx.degree, means, viewmats, coeffs,
                                             row_of, v_colors.contiguous())
        return (None, v_means if ctx.needs_input_grad[1] else None,
                v_coeffs if ctx.needs_input_grad[2] else None, None, None, None, None)


class Grad2dStatsSlot:
    """Carries a densification-statistics request from the caller to the
    packed front end's backward (``gsplat_amd.strategy.stats.fuse_grad2d_stats``
    fills it between the forward and ``backward()``): the projection backward
    then accumulates the statistics in its own pass.

    The first backward through the node consumes the request, so a second
    backward through a retained graph adds nothing; a request whose backward
    never runs adds nothing either.  The slot holds ``means2d`` (whose
    ``absgrad`` the statistics read) only weakly: the node's context holds the
    slot, and a strong reference would make means2d -> its node -> the slot
    -> means2d a cycle that keeps a step's buffers alive until Python's
    cyclic collector runs."""

    def __init__(self, width: int, height: int, n_cameras: int):
        self.scale_x = width / 2.0 * n_cameras
        self.scale_y = height / 2.0 * n_cameras
        self._means2d = None
        self.request = None  # (grad2d, count, absgrad)

    @property
    def means2d(self) -> Optional[Tensor]:
        return None if self._means2d is None else self._means2d()

    @means2d.setter
    def means2d(self, t: Optional[Tensor]) -> None:
        self._means2d = None if t is None else weakref.ref(t)


class _PackedFrontEnd(torch.autograd.Function):
    """rasterization()'s packed front end as one node: the packed projection
    (``_FullyFusedProjectionPacked``), the per-row opacities
    opacities[batch_ids, gaussian_ids] and the per-row colours (clamped SH of
    per-Gaussian coefficients, or a gather of per-Gaussian features) -- the
    reference's fully_fused_projection + index + compute_directions +
    spherical_harmonics + clamp_min (rendering.py:256-873).  The colour
    kernel runs while the host waits for the visible count
    (``_ops.packed_front_fwd``).  Backward: the colour VJP first, then one
    pass per Gaussian that writes the projection's gradients together with
    v_opacities and the colour term of v_means.  The view matrices get no
    gradient (the caller uses this node only when they need none)."""

    @staticmethod
    def forward(ctx, means, covars, quats, scales, opacities, features, viewmats,
                Ks, width, height, eps2d, near_plane, far_plane, radius_clip,
                calc_compensations, camera_model, sh_degree, isect=None,
                stats_slot=None):
        cm = _camera_model_type(camera_model)
        (indptr, batch_ids, camera_ids, gaussian_ids, radii, means2d, depths,
         conics, compensations, row_of, row_opac, row_colors) = _ops.packed_front_fwd(
            means, covars, quats, scales, opacities, features, viewmats, Ks, width,
            height, eps2d, near_plane, far_plane, radius_clip, calc_compensations,
            cm, sh_degree, isect)
        if not calc_compensations:
            compensations = None
        ctx.save_for_backward(means, covars, quats, scales, viewmats, Ks, conics,
                              compensations, row_of, features)
        ctx.set_materialize_grads(False)
        ctx.width = width
        ctx.height = height
        ctx.eps2d = eps2d
        ctx.camera_model_type = cm
        ctx.sh_degree = sh_degree
        ctx.stats_slot = stats_slot
        ctx.mark_non_differentiable(batch_ids, camera_ids, gaussian_ids, indptr, radii,
                                    row_of)
        return (batch_ids, camera_ids, gaussian_ids, indptr, radii, means2d,
                depths, conics, compensations, row_of, row_opac, row_colors)

    @staticmethod
    def backward(ctx, v_batch_ids, v_camera_ids, v_gaussian_ids, v_indptr,
                 v_radii, v_means2d, v_depths, v_conics, v_compensations, v_row_of,
                 v_row_opac, v_row_colors):
        (means, covars, quats, scales, viewmats, Ks, conics, compensations, row_of,
         features) = ctx.saved_tensors
        batch_dims = means.shape[:-2]
        N = means.shape[-2]
        C = viewmats.shape[-3]
        B = math.prod(batch_dims)
        need = ctx.needs_input_grad
        # colour VJP first: its direction term is added to v_means below
        # (for SH colours of visible rows seen by one camera, inside the
        # geometry backward's launch, gsplat_projection_packed_bwd_rows_sh:
        # config 1 115 -> 107 us, config 4 245 -> 225 us, but eight cameras
        # (config 2) 117 -> 128 us, where the geometry part's camera loop
        # dominates)
        v_features = None
        v_means_sh = None
        sh_fused = (v_row_colors is not None and (need[5] or need[0])
                    and ctx.sh_degree is not None and conics.shape[0] > 0 and C == 1)
        if v_row_colors is not None and (need[5] or need[0]) and not sh_fused:
            v_row_colors = v_row_colors.contiguous()
            if ctx.sh_degree is None:
                if need[5]:
                    v_features = _ops.rows_scatter_sum(
                        v_row_colors, row_of, B, C, N).reshape(features.shape)
            else:
                K = features.shape[-2]
                v_coeffs, v_means_sh = _ops.sh_rows_bwd(
                    ctx.sh_degree, means.reshape(B, N, 3),
                    viewmats.reshape(B, C, 4, 4), features.reshape(B, N, K, 3),
                    row_of, v_row_colors)
                v_features = v_coeffs.reshape(features.shape) if need[5] else None
                v_means_sh = v_means_sh.reshape(means.shape)
        if compensations is None:
            v_compensations = None
        elif v_compensations is not None:
            v_compensations = v_compensations.contiguous()
        v_means2d = (torch.zeros_like(conics[:, :2]) if v_means2d is None
                     else v_means2d.contiguous())
        v_conics = torch.zeros_like(conics) if v_conics is None else v_conics.contiguous()
        v_row_opac = (v_row_opac.contiguous() if v_row_opac is not None and need[4]
                      else None)
        stats = None
        slot = ctx.stats_slot
        if slot is not None and slot.request is not None:
            (grad2d, count, absgrad), slot.request = slot.request, None
            rows = v_means2d
            if absgrad:
                m2d = slot.means2d
                if m2d is None:
                    raise RuntimeError(
                        "fused densification statistics read meta['means2d'].absgrad: "
                        "keep rasterization()'s meta alive until backward() has run")
                rows = getattr(m2d, "absgrad", None)
                if rows is None:
                    raise RuntimeError("fused densification statistics need "
                                       "absgrad=True in rasterization()")
            stats = (rows.contiguous(), slot.scale_x, slot.scale_y, grad2d, count)
        if sh_fused:
            res = _ops.projection_packed_bwd_rows_sh(
                means, covars, quats, scales, viewmats, Ks, ctx.width, ctx.height,
                ctx.eps2d, ctx.camera_model_type, row_of, conics, compensations,
                v_means2d, None if v_depths is None else v_depths.contiguous(),
                v_conics, v_compensations, ctx.sh_degree, features,
                v_row_colors.contiguous(), v_row_opacities=v_row_opac, stats=stats)
            v_means, v_covars, v_quats, v_scales, v_opacities, v_coeffs = res
            v_features = v_coeffs if need[5] else None
        else:
            res = _ops.projection_packed_bwd_rows(
                means, covars, quats, scales, viewmats, Ks, ctx.width, ctx.height,
                ctx.eps2d, ctx.camera_model_type, row_of, conics, compensations,
                v_means2d, None if v_depths is None else v_depths.contiguous(),
                v_conics, v_compensations, False, v_row_opacities=v_row_opac,
                v_means_add=v_means_sh, stats=stats)
            v_means, v_covars, v_quats, v_scales = res[:4]
            v_opacities = res[5] if v_row_opac is not None else None
        return (v_means if need[0] else None,
                v_covars if need[1] else None,
                v_quats if need[2] else None,
                v_scales if need[3] else None,
                v_opacities, v_features,
                None, None, None, None, None, None, None, None, None, None, None, None,
                None)


class _RasterizeToPixels(torch.autograd.Function):
    """Tile rasterizer.  ``color_last`` (optional, one value per row): a last
    channel kept apart from ``colors`` (rasterization()'s depth channel); the
    replay kernels read and write it in place, the other path concatenates
    it."""

    @staticmethod
    def forward(ctx, means2d, conics, colors, opacities, backgrounds, masks,
                width, height, tile_size, isect_offsets, flatten_ids, absgrad,
                ed_channel=-1, color_last=None):
        # With gradients ahead the forward also keeps the replay state, so
        # the backward runs one unit per forward batch instead of one per
        # tile (the reference replays whole tiles), unless that state would
        # exceed _ops.replay_budget_bytes.
        replay = None
        ed_depth = None
        grads = any(ctx.needs_input_grad[:5]) or ctx.needs_input_grad[13]
        channels = colors.shape[-1] + (1 if color_last is not None else 0)
        if grads:
            th, tw = isect_offsets.shape[-2:]
            n_images = math.prod(isect_offsets.shape[:-2])
            replay_bytes = _ops.rasterize_replay_bytes(
                n_images, tw, th, tile_size, flatten_ids.numel(), channels)
            grads_by_replay = replay_bytes <= _ops.replay_budget_bytes
        ctx.split_last = False
        if grads and grads_by_replay:
            # the launch also zero-fills the backward's accumulators
            render_colors, render_alphas, last_ids, render_T, replay = \
                _ops.rasterize_fwd_replay(
                    means2d, conics, colors, opacities, backgrounds, masks,
                    width, height, tile_size, isect_offsets, flatten_ids,
                    expected_depth_channel=ed_channel, absgrad=absgrad,
                    color_last=color_last)
            ctx.split_last = color_last is not None
        else:
            if color_last is not None:
                colors = torch.cat([colors, color_last[..., None]], dim=-1)
            render_colors, render_alphas, last_ids, render_T = \
                _ops.rasterize_fwd_with_transmittance(
                    means2d, conics, colors, opacities, backgrounds, masks,
                    width, height, tile_size, isect_offsets, flatten_ids)
            if ed_channel >= 0:
                # the division in place (rendering.py:1259-1267); a backward
                # takes it back in torch from the divided channel
                render_colors[..., ed_channel] /= render_alphas[..., 0].clamp(min=1e-10)
                if grads:
                    ed_depth = render_colors[..., ed_channel].clone()
        ctx.save_for_backward(means2d, conics, colors, opacities, backgrounds,
                              masks, isect_offsets, flatten_ids, render_T,
                              last_ids, ed_depth,
                              color_last if ctx.split_last else None)
        ctx.has_last = color_last is not None
        # the replay records and zeroed accumulators; the accumulators are
        # consumed by the first backward (a second backward through a
        # retained graph takes fresh zeros)
        ctx.replay = replay
        ctx.ed_channel = ed_channel
        ctx.width = width
        ctx.height = height
        ctx.tile_size = tile_size
        ctx.absgrad = absgrad
        # an unused alpha (or colour) output reaches backward as None
        ctx.set_materialize_grads(False)
        return render_colors, render_alphas

    @staticmethod
    def backward(ctx, v_render_colors: Optional[Tensor],
                 v_render_alphas: Optional[Tensor]):
        (means2d, conics, colors, opacities, backgrounds, masks, isect_offsets,
         flatten_ids, render_T, last_ids, ed_depth, color_last) = ctx.saved_tensors
        if v_render_colors is None and v_render_alphas is None:
            return (None,) * 14
        channels = colors.shape[-1] + (1 if ctx.split_last else 0)
        if v_render_colors is None:
            v_render_colors = render_T.new_zeros((*render_T.shape, channels))
        v_alphas = None if v_render_alphas is None else v_render_alphas.contiguous()
        v_color_last = None
        if ctx.replay is not None:
            res = _ops.rasterize_bwd_replay(
                means2d, conics, colors, opacities, backgrounds, masks, ctx.width,
                ctx.height, ctx.tile_size, isect_offsets, flatten_ids,
                render_T, last_ids, ctx.replay, v_render_colors.contiguous(), v_alphas,
                ctx.absgrad, color_last=color_last)
            v_means2d_abs, v_means2d, v_conics, v_colors, v_opacities = res[:5]
            if ctx.split_last:
                v_color_last = res[5]
        else:
            v_rc = v_render_colors
            if ctx.ed_channel >= 0:
                # out = v / max(alpha, 1e-10): dL/dv = g / den, and the alpha
                # output gets -(g / den) out where the clamp passes
                alpha = 1.0 - render_T
                gd = v_render_colors[..., ctx.ed_channel] / alpha.clamp(min=1e-10)
                v_rc = v_render_colors.clone()
                v_rc[..., ctx.ed_channel] = gd
                v_a = (-(gd * ed_depth) * (alpha >= 1e-10))[..., None]
                v_alphas = (v_a if v_alphas is None else v_alphas + v_a).contiguous()
            # render_alphas = 1 - T is only read when T is absent; T's storage
            # stands in for it to satisfy the op's checks
            (v_means2d_abs, v_means2d, v_conics, v_colors,
             v_opacities) = _ops.rasterize_to_pixels_3dgs_bwd(
                means2d, conics, colors, opacities, backgrounds, masks, ctx.width,
                ctx.height, ctx.tile_size, isect_offsets, flatten_ids,
                render_T, last_ids, v_rc.contiguous(), v_alphas,
                ctx.absgrad, render_transmittance=render_T)
        if ctx.absgrad:
            prev = getattr(means2d, "absgrad", None)
            if prev is not None and getattr(means2d, "_absgrad_pass", None) is \
                    torch._C._current_graph_task_id():
                v_means2d_abs = prev + v_means2d_abs
            means2d.absgrad = v_means2d_abs
            means2d._absgrad_pass = torch._C._current_graph_task_id()
        if ctx.needs_input_grad[4]:
            v_bg_colors = v_render_colors
            if ctx.ed_channel >= 0:
                # the divided channel: d out / d background = T / max(alpha, 1e-10)
                v_bg_colors = v_render_colors.clone()
                v_bg_colors[..., ctx.ed_channel] /= (1.0 - render_T).clamp(min=1e-10)
            v_backgrounds = (v_bg_colors * render_T[..., None]).sum(
                dim=(-3, -2))
        else:
            v_backgrounds = None
        if ctx.has_last and not ctx.split_last:
            # the concatenated colours' gradient, split back
            v_color_last = v_colors[..., -1]
            v_colors = v_colors[..., :-1]
        return (v_means2d, v_conics, v_colors, v_opacities, v_backgrounds,
                None, None, None, None, None, None, None, None, v_color_last)
