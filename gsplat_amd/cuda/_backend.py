"""Registers the ``torch.ops.gsplat`` operators backed by libgsplat_hip.so.

The schemas are the reference's, verbatim (gsplat/cuda/ext.cpp:711-754), and
the implementations are registered for the CUDA dispatch key, which is the HIP
device on ROCm builds of PyTorch (the reference registers its kernels the same
way, gsplat/cuda/ext.cpp:772-808).  No CPU kernel is registered: calling an op
with host tensors raises, as the reference does.

``_C`` stands in for the reference's compiled module (gsplat/cuda/_backend.py,
``_C``): importing it guarantees the ops are registered, and it exposes the
``CameraModelType`` enum (gsplat/cuda/ext.cpp:38-44).
"""

from __future__ import annotations

import enum
import types

import torch

from .. import _lib
from . import _ops


class CameraModelType(enum.IntEnum):
    PINHOLE = 0
    ORTHO = 1
    FISHEYE = 2
    FTHETA = 3
    LIDAR = 4


_SCHEMAS = {
    "spherical_harmonics_fwd":
        "spherical_harmonics_fwd(int degrees_to_use, Tensor dirs, Tensor coeffs, "
        "Tensor? masks) -> Tensor",
    "spherical_harmonics_bwd":
        "spherical_harmonics_bwd(int degrees_to_use, Tensor dirs, Tensor coeffs, "
        "Tensor? masks, Tensor v_colors, bool compute_v_dirs) -> (Tensor, Tensor)",
    "intersect_tile":
        "intersect_tile(Tensor means2d, Tensor radii, Tensor depths, Tensor? conics, "
        "Tensor? opacities, Tensor? image_ids, Tensor? gaussian_ids, int I, "
        "int tile_size, int tile_width, int tile_height, bool sort, bool segmented) "
        "-> (Tensor, Tensor, Tensor)",
    "intersect_offset":
        "intersect_offset(Tensor isect_ids, int I, int tile_width, int tile_height) "
        "-> Tensor",
    "projection_ewa_3dgs_fused_fwd":
        "projection_ewa_3dgs_fused_fwd(Tensor means, Tensor? covars, Tensor? quats, "
        "Tensor? scales, Tensor? opacities, Tensor viewmats, Tensor Ks, "
        "int image_width, int image_height, float eps2d, float near_plane, "
        "float far_plane, float radius_clip, bool calc_compensations, "
        "int camera_model) -> (Tensor, Tensor, Tensor, Tensor, Tensor)",
    "projection_ewa_3dgs_fused_bwd":
        "projection_ewa_3dgs_fused_bwd(Tensor means, Tensor? covars, Tensor? quats, "
        "Tensor? scales, Tensor viewmats, Tensor Ks, int image_width, "
        "int image_height, float eps2d, int camera_model, Tensor radii, "
        "Tensor conics, Tensor? compensations, Tensor v_means2d, Tensor v_depths, "
        "Tensor v_conics, Tensor? v_compensations, bool viewmats_requires_grad) "
        "-> (Tensor, Tensor, Tensor, Tensor, Tensor)",
    "projection_ewa_3dgs_packed_fwd":
        "projection_ewa_3dgs_packed_fwd(Tensor means, Tensor? covars, Tensor? quats, "
        "Tensor? scales, Tensor? opacities, Tensor viewmats, Tensor Ks, "
        "int image_width, int image_height, float eps2d, float near_plane, "
        "float far_plane, float radius_clip, bool calc_compensations, "
        "int camera_model) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, "
        "Tensor, Tensor, Tensor)",
    "projection_ewa_3dgs_packed_bwd":
        "projection_ewa_3dgs_packed_bwd(Tensor means, Tensor? covars, Tensor? quats, "
        "Tensor? scales, Tensor viewmats, Tensor Ks, int image_width, "
        "int image_height, float eps2d, int camera_model, Tensor batch_ids, "
        "Tensor camera_ids, Tensor gaussian_ids, Tensor conics, "
        "Tensor? compensations, Tensor v_means2d, Tensor v_depths, Tensor v_conics, "
        "Tensor? v_compensations, bool viewmats_requires_grad, bool sparse_grad) "
        "-> (Tensor, Tensor, Tensor, Tensor, Tensor)",
    "rasterize_to_pixels_3dgs_fwd":
        "rasterize_to_pixels_3dgs_fwd(Tensor means2d, Tensor conics, Tensor colors, "
        "Tensor opacities, Tensor? backgrounds, Tensor? masks, int image_width, "
        "int image_height, int tile_size, Tensor tile_offsets, Tensor flatten_ids) "
        "-> (Tensor, Tensor, Tensor)",
    "rasterize_to_pixels_3dgs_bwd":
        "rasterize_to_pixels_3dgs_bwd(Tensor means2d, Tensor conics, Tensor colors, "
        "Tensor opacities, Tensor? backgrounds, Tensor? masks, int image_width, "
        "int image_height, int tile_size, Tensor tile_offsets, Tensor flatten_ids, "
        "Tensor render_alphas, Tensor last_ids, Tensor v_render_colors, "
        "Tensor v_render_alphas, bool absgrad) -> (Tensor, Tensor, Tensor, Tensor, "
        "Tensor)",
    "adam":
        "adam(Tensor(a!) param, Tensor param_grad, Tensor(b!) exp_avg, "
        "Tensor(c!) exp_avg_sq, Tensor? valid, float lr, float b1, float b2, "
        "float eps) -> ()",
}


def _undef(like: torch.Tensor):
    # stand-in for the reference's undefined optional outputs
    return torch.empty(0, dtype=torch.float32, device=like.device)


def _fill(outs, like):
    return tuple(o if o is not None else _undef(like) for o in outs)


def _impl_sh_bwd(deg, dirs, coeffs, masks, v_colors, compute_v_dirs):
    return _fill(_ops.spherical_harmonics_bwd(deg, dirs, coeffs, masks, v_colors,
                                              compute_v_dirs), dirs)


def _impl_fused_fwd(*args):
    return _fill(_ops.projection_ewa_3dgs_fused_fwd(*args), args[0])


def _impl_fused_bwd(*args):
    return _fill(_ops.projection_ewa_3dgs_fused_bwd(*args), args[0])


def _impl_packed_fwd(*args):
    return _fill(_ops.projection_ewa_3dgs_packed_fwd(*args), args[0])


def _impl_packed_bwd(*args):
    return _fill(_ops.projection_ewa_3dgs_packed_bwd(*args), args[0])


def _impl_raster_bwd(*args):
    return _fill(_ops.rasterize_to_pixels_3dgs_bwd(*args), args[0])


_IMPLS = {
    "spherical_harmonics_fwd": _ops.spherical_harmonics_fwd,
    "spherical_harmonics_bwd": _impl_sh_bwd,
    "intersect_tile": _ops.intersect_tile,
    "intersect_offset": _ops.intersect_offset,
    "projection_ewa_3dgs_fused_fwd": _impl_fused_fwd,
    "projection_ewa_3dgs_fused_bwd": _impl_fused_bwd,
    "projection_ewa_3dgs_packed_fwd": _impl_packed_fwd,
    "projection_ewa_3dgs_packed_bwd": _impl_packed_bwd,
    "rasterize_to_pixels_3dgs_fwd": _ops.rasterize_to_pixels_3dgs_fwd,
    "rasterize_to_pixels_3dgs_bwd": _impl_raster_bwd,
    "adam": _ops.adam,
}

_SCHEMAS.update({
    "projection_ewa_simple_fwd":
        "projection_ewa_simple_fwd(Tensor means, Tensor covars, Tensor Ks, int width, "
        "int height, int camera_model) -> (Tensor, Tensor)",
    "projection_ewa_simple_bwd":
        "projection_ewa_simple_bwd(Tensor means, Tensor covars, Tensor Ks, int width, "
        "int height, int camera_model, Tensor v_means2d, Tensor v_covars2d) "
        "-> (Tensor, Tensor)",
})
_IMPLS.update({
    "projection_ewa_simple_fwd": _ops.projection_ewa_simple_fwd,
    "projection_ewa_simple_bwd": _ops.projection_ewa_simple_bwd,
})

_SCHEMAS.update({
    "quat_scale_to_covar_preci_fwd":
        "quat_scale_to_covar_preci_fwd(Tensor quats, Tensor scales, bool compute_covar, "
        "bool compute_preci, bool triu) -> (Tensor, Tensor)",
    "quat_scale_to_covar_preci_bwd":
        "quat_scale_to_covar_preci_bwd(Tensor quats, Tensor scales, bool triu, "
        "Tensor? v_covars, Tensor? v_precis) -> (Tensor, Tensor)",
    "rasterize_to_indices_3dgs":
        "rasterize_to_indices_3dgs(int range_start, int range_end, Tensor transmittances, "
        "Tensor means2d, Tensor conics, Tensor opacities, int image_width, "
        "int image_height, int tile_size, Tensor tile_offsets, Tensor flatten_ids) "
        "-> (Tensor, Tensor)",
})


def _impl_covar_fwd(quats, scales, compute_covar, compute_preci, triu):
    return _fill(_ops.quat_scale_to_covar_preci_fwd(quats, scales, compute_covar,
                                                    compute_preci, triu), quats)


_IMPLS.update({
    "quat_scale_to_covar_preci_fwd": _impl_covar_fwd,
    "quat_scale_to_covar_preci_bwd": _ops.quat_scale_to_covar_preci_bwd,
    "rasterize_to_indices_3dgs": _ops.rasterize_to_indices_3dgs,
})

_LIBRARY = None


def _register() -> None:
    global _LIBRARY
    if _LIBRARY is not None:
        return
    lib = torch.library.Library("gsplat", "DEF")
    for name, schema in _SCHEMAS.items():
        lib.define(schema)
        lib.impl(name, _IMPLS[name], "CUDA")
    _LIBRARY = lib


_register()
_lib.load()

# Stand-in for the reference's compiled extension module.
_C = types.SimpleNamespace(CameraModelType=CameraModelType, lib=_lib)
