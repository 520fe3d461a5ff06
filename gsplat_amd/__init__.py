"""gsplat_amd: MI355X-native (gfx950 HIP) kernels for gsplat's differentiable
3D Gaussian splatting hot path, behind the reference's Python API.

    import gsplat_amd as gsplat
    colors, alphas, meta = gsplat.rasterization(means, quats, scales, opacities,
                                                colors, viewmats, Ks, W, H)
"""

from .cuda._wrapper import (
    adam,
    fully_fused_projection,
    has_2dgs,
    has_3dgs,
    has_3dgut,
    has_adam,
    has_camera_wrappers,
    has_reloc,
    isect_offset_encode,
    isect_tiles,
    proj,
    quat_scale_to_covar_preci,
    rasterize_to_indices_in_range,
    rasterize_to_pixels,
    spherical_harmonics,
)
from .optimizers import SelectiveAdam
from .rendering import rasterization
from .strategy.stats import accumulate_grad2d_stats

__version__ = "0.1.0"

__all__ = [
    "adam",
    "accumulate_grad2d_stats",
    "fully_fused_projection",
    "has_2dgs",
    "has_3dgs",
    "has_3dgut",
    "has_adam",
    "has_camera_wrappers",
    "has_reloc",
    "isect_offset_encode",
    "isect_tiles",
    "proj",
    "quat_scale_to_covar_preci",
    "rasterization",
    "rasterize_to_indices_in_range",
    "rasterize_to_pixels",
    "spherical_harmonics",
    "SelectiveAdam",
]
