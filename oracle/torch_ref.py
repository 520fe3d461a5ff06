"""Float restatement of the splatting math in PyTorch (TEST INFRASTRUCTURE ONLY).

Runs on the CPU in float32 or float64; gradients come from autograd, so they
check the hand-derived HIP backward kernels independently.  Sources:
  projection  gsplat/cuda/_torch_impl.py:214-340 (+ the opacity-aware radius
              and culling of ProjectionEWA3DGSFused.cu:186-220),
              gsplat/cuda/_math.py:649-713;
  SH          gsplat/cuda/_torch_impl.py:686-788;
  rasterizer  gsplat/cuda/_torch_impl.py:472-683 with the compositing rules of
              RasterizeToPixels3DGSFwd.cu:140-212;
  pipeline    gsplat/rendering.py:256-1273 (3DGS path).
Discrete decisions (which rows are visible, which tiles a row touches, which
pixel/Gaussian pairs are composited) are taken from the bit-exact oracle in
``exact`` so they are identical to the GPU's; the continuous values that feed
them come from this module with autograd.
"""

from __future__ import annotations

import math
from typing import Dict, Optional

import numpy as np
import torch
import torch.nn.functional as F
from torch import Tensor

from . import exact

ALPHA_THRESHOLD = 1.0 / 255.0
MAX_ALPHA = 0.99
TRANSMITTANCE_THRESHOLD = 1e-4
MIN_COMPENSATION = 0.005


# --------------------------------------------------------------------------
# Geometry
# --------------------------------------------------------------------------
def quat_to_rotmat(quats: Tensor) -> Tensor:
    """Rotation matrix of (w, x, y, z) quaternions (gsplat/cuda/_math.py:649-669)."""
    q = F.normalize(quats, p=2, dim=-1)
    w, x, y, z = torch.unbind(q, dim=-1)
    R = torch.stack([
        1 - 2 * (y ** 2 + z ** 2), 2 * (x * y - w * z), 2 * (x * z + w * y),
        2 * (x * y + w * z), 1 - 2 * (x ** 2 + z ** 2), 2 * (y * z - w * x),
        2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x ** 2 + y ** 2),
    ], dim=-1)
    return R.reshape(quats.shape[:-1] + (3, 3))


def quat_scale_to_covar(quats: Tensor, scales: Tensor) -> Tensor:
    """Sigma = R S S R^T (gsplat/cuda/_math.py:683-713)."""
    R = quat_to_rotmat(quats)
    M = R * scales[..., None, :]
    return M @ M.transpose(-1, -2)


def camera_centers(viewmats: Tensor) -> Tensor:
    """World position -R^T t of the camera of each world->camera matrix
    [..., 4, 4] (gsplat/rendering.py:216-224); the SH view direction of a
    Gaussian is its mean minus this point (rendering.py:227-253)."""
    R = viewmats[..., :3, :3]
    t = viewmats[..., :3, 3:]
    return -(R.transpose(-1, -2) @ t)[..., 0]


def covar6_to_mat(c6: Tensor) -> Tensor:
    a, b, c, d, e, f = torch.unbind(c6, dim=-1)
    return torch.stack([a, b, c, b, d, e, c, e, f], dim=-1).reshape(c6.shape[:-1] + (3, 3))


def proj_ref(means, covars, Ks, width, height, camera_model="pinhole"):
    """Camera-space projection of Gaussians, differentiable: means [..., C, N, 3],
    covars [..., C, N, 3, 3] -> means2d [..., C, N, 2], cov2d = J S J^T
    [..., C, N, 2, 2] (gsplat/cuda/_torch_impl.py:42-97 pinhole with the
    1.3x field-of-view clamp of the Jacobian, :169-211 orthographic)."""
    x, y, z = torch.unbind(means, dim=-1)
    fx = Ks[..., 0, 0, None]
    fy = Ks[..., 1, 1, None]
    cx = Ks[..., 0, 2, None]
    cy = Ks[..., 1, 2, None]
    zero = torch.zeros_like(z)
    if camera_model == "ortho":
        J = torch.stack([fx + zero, zero, zero, zero, fy + zero, zero], dim=-1)
        means2d = torch.stack([fx * x + cx, fy * y + cy], dim=-1)
    else:
        tan_fovx = 0.5 * width / fx
        tan_fovy = 0.5 * height / fy
        lim_x_pos = (width - cx) / fx + 0.3 * tan_fovx
        lim_x_neg = cx / fx + 0.3 * tan_fovx
        lim_y_pos = (height - cy) / fy + 0.3 * tan_fovy
        lim_y_neg = cy / fy + 0.3 * tan_fovy
        tx = z * torch.minimum(lim_x_pos, torch.maximum(-lim_x_neg, x / z))
        ty = z * torch.minimum(lim_y_pos, torch.maximum(-lim_y_neg, y / z))
        J = torch.stack([fx / z, zero, -fx * tx / z ** 2,
                         zero, fy / z, -fy * ty / z ** 2], dim=-1)
        means2d = torch.stack([fx * x / z + cx, fy * y / z + cy], dim=-1)
    J = J.reshape(J.shape[:-1] + (2, 3))
    return means2d, J @ covars @ J.transpose(-1, -2)


def projection_ref(means, covars, quats, scales, viewmats, Ks, width, height,
                   eps2d=0.3, near_plane=0.01, far_plane=1e10, radius_clip=0.0,
                   calc_compensations=False, camera_model="pinhole",
                   opacities=None) -> Dict[str, Tensor]:
    """Dense EWA projection of [..., C, N] rows (differentiable).

    Returns means2d, depths, conics, compensations and the float radius
    estimate / visibility test of this float formulation ("radius_f",
    "valid")."""
    if covars is not None:
        Sigma = covar6_to_mat(covars)
    else:
        Sigma = quat_scale_to_covar(quats, scales)
    R = viewmats[..., :3, :3]
    t = viewmats[..., :3, 3]
    means_c = torch.einsum("...cij,...nj->...cni", R, means) + t[..., None, :]
    covars_c = torch.einsum("...cij,...njk,...clk->...cnil", R, Sigma, R)
    x, y, z = torch.unbind(means_c, dim=-1)
    fx = Ks[..., 0, 0, None]
    fy = Ks[..., 1, 1, None]
    cx = Ks[..., 0, 2, None]
    cy = Ks[..., 1, 2, None]
    zero = torch.zeros_like(z)
    if camera_model == "ortho":
        J = torch.stack([fx + zero, zero, zero, zero, fy + zero, zero], dim=-1)
        means2d = torch.stack([fx * x + cx, fy * y + cy], dim=-1)
    else:
        tan_fovx = 0.5 * width / fx
        tan_fovy = 0.5 * height / fy
        lim_x_pos = (width - cx) / fx + 0.3 * tan_fovx
        lim_x_neg = cx / fx + 0.3 * tan_fovx
        lim_y_pos = (height - cy) / fy + 0.3 * tan_fovy
        lim_y_neg = cy / fy + 0.3 * tan_fovy
        tx = z * torch.minimum(lim_x_pos, torch.maximum(-lim_x_neg, x / z))
        ty = z * torch.minimum(lim_y_pos, torch.maximum(-lim_y_neg, y / z))
        J = torch.stack([fx / z, zero, -fx * tx / z ** 2,
                         zero, fy / z, -fy * ty / z ** 2], dim=-1)
        means2d = torch.stack([fx * x / z + cx, fy * y / z + cy], dim=-1)
    J = J.reshape(J.shape[:-1] + (2, 3))
    cov2d = J @ covars_c @ J.transpose(-1, -2)
    det_orig = cov2d[..., 0, 0] * cov2d[..., 1, 1] - cov2d[..., 0, 1] * cov2d[..., 1, 0]
    c00 = cov2d[..., 0, 0] + eps2d
    c11 = cov2d[..., 1, 1] + eps2d
    c01 = 0.5 * (cov2d[..., 0, 1] + cov2d[..., 1, 0])
    det = c00 * c11 - c01 * c01
    det_safe = torch.where(det > 0, det, torch.ones_like(det))
    comp = torch.sqrt(torch.clamp(det_orig / det_safe, min=MIN_COMPENSATION ** 2))
    conics = torch.stack([c11 / det_safe, -c01 / det_safe, c00 / det_safe], dim=-1)
    depths = z
    with torch.no_grad():
        valid = (z >= near_plane) & (z <= far_plane) & (det > 0)
        extend = torch.full_like(z, 3.33)
        if opacities is not None:
            op = torch.broadcast_to(opacities[..., None, :], z.shape)
            if calc_compensations:
                op = op * comp
            valid &= op >= ALPHA_THRESHOLD
            extend = torch.clamp(torch.sqrt(2.0 * torch.log(
                torch.clamp(op, min=1e-30) / ALPHA_THRESHOLD).clamp(min=0)), max=3.33)
        rx = torch.ceil(extend * torch.sqrt(c00.clamp(min=0)))
        ry = torch.ceil(extend * torch.sqrt(c11.clamp(min=0)))
        valid &= ~((rx <= radius_clip) & (ry <= radius_clip))
        mx, my = means2d[..., 0], means2d[..., 1]
        valid &= ~((mx + rx <= 0) | (mx - rx >= width) | (my + ry <= 0) | (my - ry >= height))
    return {
        "means2d": means2d, "depths": depths, "conics": conics,
        "compensations": comp if calc_compensations else None,
        "radius_f": torch.stack([rx, ry], dim=-1), "valid": valid,
        "extend_arg": c00,
    }


# --------------------------------------------------------------------------
# Spherical harmonics
# --------------------------------------------------------------------------
def sh_bases(basis_dim: int, dirs: Tensor) -> Tensor:
    """Real SH basis (Sloan 2013) at unit directions
    (gsplat/cuda/_torch_impl.py:686-768)."""
    out = torch.zeros(dirs.shape[:-1] + (basis_dim,), dtype=dirs.dtype)
    cols = [torch.full(dirs.shape[:-1], 0.2820947917738781, dtype=dirs.dtype)]
    if basis_dim > 1:
        x, y, z = dirs.unbind(-1)
        a = 0.48860251190292
        cols += [-a * y, a * z, -a * x]
    if basis_dim > 4:
        z2 = z * z
        fC1 = x * x - y * y
        fS1 = 2 * x * y
        tB = -1.092548430592079 * z
        cols += [0.5462742152960395 * fS1, tB * y,
                 0.9461746957575601 * z2 - 0.3153915652525201, tB * x,
                 0.5462742152960395 * fC1]
    if basis_dim > 9:
        tC = -2.285228997322329 * z2 + 0.4570457994644658
        tB3 = 1.445305721320277 * z
        fC2 = x * fC1 - y * fS1
        fS2 = x * fS1 + y * fC1
        cols += [-0.5900435899266435 * fS2, tB3 * fS1, tC * y,
                 z * (1.865881662950577 * z2 - 1.119528997770346), tC * x,
                 tB3 * fC1, -0.5900435899266435 * fC2]
    if basis_dim > 16:
        tD = z * (-4.683325804901025 * z2 + 2.007139630671868)
        tC4 = 3.31161143515146 * z2 - 0.47308734787878
        tB4 = -1.770130769779931 * z
        fC3 = x * fC2 - y * fS2
        fS3 = x * fS2 + y * fC2
        y12 = z * (1.865881662950577 * z2 - 1.119528997770346)
        y6 = 0.9461746957575601 * z2 - 0.3153915652525201
        cols += [0.6258357354491763 * fS3, tB4 * fS2, tC4 * fS1, tD * y,
                 1.984313483298443 * z * y12 - 1.006230589874905 * y6, tD * x,
                 tC4 * fC1, tB4 * fC2, 0.6258357354491763 * fC3]
    return torch.stack(cols[:basis_dim], dim=-1)


def spherical_harmonics_ref(degree: int, dirs: Tensor, coeffs: Tensor,
                            masks: Optional[Tensor] = None) -> Tensor:
    """colors = sum_k Y_k(dir/|dir|) coeffs[k] (masked rows -> 0)."""
    nb = (degree + 1) ** 2
    d = dirs / torch.linalg.norm(dirs, dim=-1, keepdim=True)
    Y = sh_bases(nb, d)
    colors = (Y[..., None] * coeffs[..., :nb, :]).sum(dim=-2)
    if masks is not None:
        colors = torch.where(masks[..., None], colors, torch.zeros_like(colors))
    return colors


# --------------------------------------------------------------------------
# Tile rasterizer
# --------------------------------------------------------------------------
def rasterize_to_pixels_ref(means2d, conics, colors, opacities, width, height,
                            tile_size, isect_offsets, flatten_ids,
                            backgrounds=None, masks=None, decide=None,
                            dtype=torch.float64):
    """Front-to-back compositing per tile, differentiable.

    means2d [..., N, 2] or [nnz, 2] (rows are what ``flatten_ids`` index);
    ``decide``: optional dict with float32 numpy ``means2d``, ``conics``,
    ``opacities`` (flattened rows) used for the discrete decisions; by default
    the float32 values of the inputs.

    Returns (render_colors [I, H, W, D], render_alphas [I, H, W, 1], info)
    where info holds ``last_ids`` [I, H, W] and ``transmittance`` [I, H, W]
    (the float32 running transmittance at the end of each pixel's list).

    Which Gaussians a pixel composites, and where it stops, is decided in
    float32 exactly as the kernels do: sigma in the kernels' operation order,
    alpha = o * portable_expf(-sigma) (bit-identical to the device), T a
    running float32 product, stop before the first Gaussian with
    T (1 - alpha) <= 1e-4.  The differentiable values use ``dtype``.
    """
    th, tw = isect_offsets.shape[-2:]
    I = int(np.prod(isect_offsets.shape[:-2])) if isect_offsets.dim() > 2 else 1
    D = colors.shape[-1]
    xy = means2d.reshape(-1, 2).to(dtype)
    con = conics.reshape(-1, 3).to(dtype)
    op = opacities.reshape(-1).to(dtype)
    col = colors.reshape(-1, D).to(dtype)
    bgs = backgrounds.reshape(I, D).to(dtype) if backgrounds is not None else None
    if decide is None:
        decide = {
            "means2d": means2d.detach().reshape(-1, 2).float().numpy(),
            "conics": conics.detach().reshape(-1, 3).float().numpy(),
            "opacities": opacities.detach().reshape(-1).float().numpy(),
        }
    xy32 = np.ascontiguousarray(decide["means2d"], np.float32).reshape(-1, 2)
    con32 = np.ascontiguousarray(decide["conics"], np.float32).reshape(-1, 3)
    sig_max, sig_clamp = exact.alpha_thresholds(np.asarray(decide["opacities"], np.float32).reshape(-1))
    offs = isect_offsets.reshape(-1).cpu().numpy().astype(np.int64)
    fids = flatten_ids.cpu().numpy().astype(np.int64)
    n_isects = fids.shape[0]
    ends = np.append(offs[1:], n_isects)
    mask_np = masks.reshape(-1).cpu().numpy() if masks is not None else None

    pix_index, pix_colors, pix_alphas = [], [], []
    last_ids = np.zeros(I * height * width, np.int32)
    trans = np.ones(I * height * width, np.float32)
    for slot in range(I * th * tw):
        img = slot // (th * tw)
        tile = slot % (th * tw)
        ty, tx = tile // tw, tile % tw
        ys = np.arange(ty * tile_size, min((ty + 1) * tile_size, height))
        xs = np.arange(tx * tile_size, min((tx + 1) * tile_size, width))
        if ys.size == 0 or xs.size == 0:
            continue
        yy, xx = np.meshgrid(ys, xs, indexing="ij")
        yy, xx = yy.ravel(), xx.ravel()
        lin = img * height * width + yy * width + xx
        P = lin.size
        bg = bgs[img] if bgs is not None else torch.zeros(D, dtype=dtype)
        s, e = offs[slot], ends[slot]
        if (mask_np is not None and not mask_np[slot]) or e <= s:
            pix_index.append(lin)
            pix_colors.append(bg[None, :].expand(P, D))
            pix_alphas.append(torch.zeros(P, dtype=dtype))
            continue
        ids = fids[s:e]
        n = ids.size
        px32 = xx.astype(np.float32) + np.float32(0.5)
        py32 = yy.astype(np.float32) + np.float32(0.5)
        dx32 = xy32[ids, 0][None, :] - px32[:, None]
        dy32 = xy32[ids, 1][None, :] - py32[:, None]
        sig32 = exact.gauss_sigma_f32(con32[ids, 0][None, :], con32[ids, 1][None, :],
                                      con32[ids, 2][None, :], dx32, dy32)
        skip = (sig32 < 0) | (sig32 > sig_max[ids][None, :])
        clamped = sig32 < sig_clamp[ids][None, :]
        idt = torch.from_numpy(ids)
        pxt = torch.from_numpy(px32.astype(np.float64)).to(dtype)
        pyt = torch.from_numpy(py32.astype(np.float64)).to(dtype)
        g_xy = xy[idt]
        g_con = con[idt]
        dx = g_xy[None, :, 0] - pxt[:, None]
        dy = g_xy[None, :, 1] - pyt[:, None]
        sigma = 0.5 * (g_con[None, :, 0] * dx * dx + g_con[None, :, 2] * dy * dy) \
            + g_con[None, :, 1] * dx * dy
        skip_t = torch.from_numpy(skip)
        clamp_t = torch.from_numpy(clamped)
        a_raw = op[idt][None, :] * torch.exp(-sigma)
        alpha = torch.where(skip_t, torch.zeros_like(a_raw),
                            torch.where(clamp_t, torch.full_like(a_raw, MAX_ALPHA), a_raw))
        # Decisions in float32 with the device's exact alpha (see docstring).
        o32 = np.asarray(decide["opacities"], np.float32).reshape(-1)[ids][None, :]
        with np.errstate(over="ignore", invalid="ignore"):
            vis32 = exact.portable_expf(-sig32)
            a32 = np.where(skip, np.float32(0.0),
                           np.where(clamped, exact.MAX_ALPHA, (o32 * vis32).astype(np.float32)))
        one_m32 = (np.float32(1.0) - a32).astype(np.float32)
        Tb32 = np.cumprod(np.concatenate([np.ones((P, 1), np.float32), one_m32[:, :-1]],
                                         axis=1), axis=1, dtype=np.float32)
        next32 = (Tb32 * one_m32).astype(np.float32)
        cand = (~skip) & (next32 <= exact.TRANSMITTANCE_THRESHOLD)
        has = cand.any(axis=1)
        k_stop = np.where(has, cand.argmax(axis=1), n)
        ar = np.arange(n)[None, :]
        included_np = (ar < k_stop[:, None]) & ~skip
        # float32 transmittance after the last composited Gaussian
        T_end32 = np.where(has, Tb32[np.arange(P), np.minimum(k_stop, n - 1)],
                           next32[:, -1] if n > 0 else np.ones(P, np.float32))
        last_np = np.where(included_np, ar, -1).max(axis=1)
        included = torch.from_numpy(included_np)
        ai = alpha * included.to(dtype)
        Tcum = torch.cumprod(torch.cat([torch.ones(P, 1, dtype=dtype), 1.0 - ai[:, :-1]],
                                       dim=1), dim=1)
        w = ai * Tcum
        T_final = Tcum[:, -1] * (1.0 - ai[:, -1])
        c = w @ col[idt] + T_final[:, None] * bg[None, :]
        pix_index.append(lin)
        pix_colors.append(c)
        pix_alphas.append(1.0 - T_final)
        last_ids[lin] = np.where(last_np >= 0, s + last_np, 0)
        trans[lin] = T_end32
    idx = torch.from_numpy(np.concatenate(pix_index))
    out_c = torch.zeros(I * height * width, D, dtype=dtype).index_copy(
        0, idx, torch.cat(pix_colors, dim=0))
    out_a = torch.zeros(I * height * width, dtype=dtype).index_copy(
        0, idx, torch.cat(pix_alphas, dim=0))
    info = {
        "last_ids": last_ids.reshape(I, height, width),
        "transmittance": trans.reshape(I, height, width),
    }
    return (out_c.reshape(I, height, width, D), out_a.reshape(I, height, width, 1), info)


# --------------------------------------------------------------------------
# Full rasterization() pipeline (3DGS path)
# --------------------------------------------------------------------------
def rasterization_ref(means, quats, scales, opacities, colors, viewmats, Ks,
                      width, height, near_plane=0.01, far_plane=1e10,
                      radius_clip=0.0, eps2d=0.3, sh_degree=None, packed=True,
                      tile_size=16, backgrounds=None, render_mode="RGB",
                      rasterize_mode="classic", camera_model="pinhole",
                      dtype=torch.float64, tile_subset=None, restrict_rows=False):
    """CPU restatement of ``rasterization()`` for one batch (no batch dims).

    Inputs are CPU tensors (float32 values; gradients flow to them).  The
    visible rows, their tile lists and sorted order come from the bit-exact
    oracle run on the float32 inputs; the differentiable values from
    ``projection_ref`` in ``dtype``.  ``tile_subset`` (optional iterable of
    tile slots) restricts the rasterizer to a sample of tiles; other tiles are
    left empty.  With ``restrict_rows`` the float restatement (projection,
    SH) is evaluated only on the rows those tiles reference, which bounds the
    cost of checking full-size scenes; the values are the same either way.
    Returns (render_colors, render_alphas, meta).
    """
    N = means.shape[-2]
    C = viewmats.shape[-3]
    calc_comp = rasterize_mode == "antialiased"
    cm = {"pinhole": 0, "ortho": 1}[camera_model]
    f32 = lambda t: None if t is None else t.detach().float().numpy()
    ex = exact.projection_fwd(f32(means), None, f32(quats), f32(scales), f32(opacities),
                              f32(viewmats), f32(Ks), width, height, eps2d, near_plane,
                              far_plane, radius_clip, calc_comp, cm)
    valid = ex["valid"].reshape(C * N)
    # float32 values the GPU sees (bit-exact oracle) for the decisions
    ex_op = np.broadcast_to(f32(opacities)[None, :], (C, N)).reshape(C * N)
    if calc_comp:
        ex_op = (ex_op * ex["compensations"].reshape(C * N)).astype(np.float32)
    ex_m2 = ex["means2d"].reshape(C * N, 2)
    ex_con = ex["conics"].reshape(C * N, 3)
    ex_dep = ex["depths"].reshape(C * N)
    ex_rad = ex["radii"].reshape(C * N, 2)

    tile_w = math.ceil(width / tile_size)
    tile_h = math.ceil(height / tile_size)
    if packed:
        # rows: the flattened (camera, Gaussian) index of each packed row
        rows = np.nonzero(valid)[0]
        image_ids = (rows // N).astype(np.int64)
        _, isect_ids, flatten_ids = exact.isect_tiles(
            ex_m2[rows], ex_rad[rows], ex_dep[rows], tile_size, tile_w, tile_h,
            packed=True, n_images=C, image_ids=image_ids, conics=ex_con[rows],
            opacities=ex_op[rows])
    else:
        rows = np.arange(C * N)
        _, isect_ids, flatten_ids = exact.isect_tiles(
            ex_m2.reshape(C, N, 2), ex_rad.reshape(C, N, 2), ex_dep.reshape(C, N),
            tile_size, tile_w, tile_h, conics=ex_con.reshape(C, N, 3),
            opacities=ex_op.reshape(C, N))
    offsets = exact.isect_offset_encode(isect_ids, C, tile_w, tile_h)
    masks = None
    fl = flatten_ids
    if tile_subset is not None:
        sub = np.unique(np.asarray(list(tile_subset), np.int64))
        m = np.zeros(C * tile_h * tile_w, bool)
        m[sub] = True
        masks = torch.from_numpy(m.reshape(C, tile_h, tile_w))
    if tile_subset is not None and restrict_rows:
        offs = offsets.reshape(-1).astype(np.int64)
        ends = np.append(offs[1:], flatten_ids.shape[0])
        used = np.unique(np.concatenate(
            [flatten_ids[offs[t]:ends[t]] for t in sub] + [np.zeros(0, np.int32)]))
        lookup = np.zeros(rows.shape[0], np.int32)
        lookup[used] = np.arange(used.shape[0], dtype=np.int32)
        fl = lookup[flatten_ids]
        need = used.astype(np.int64)
    else:
        need = np.arange(rows.shape[0], dtype=np.int64)
    # the differentiable values of the needed rows, one camera at a time
    flat_need = rows[need]
    cam_need, gid_need = flat_need // N, flat_need % N
    n_need = need.shape[0]
    m2_rows = torch.zeros(n_need, 2, dtype=dtype)
    con_rows = torch.zeros(n_need, 3, dtype=dtype)
    dep_rows = torch.zeros(n_need, dtype=dtype)
    comp_rows = torch.zeros(n_need, dtype=dtype) if calc_comp else None
    feat_parts = []
    if sh_degree is not None:
        campos = camera_centers(viewmats.to(dtype))
    for c in range(C):
        sel_c = np.nonzero(cam_need == c)[0]
        if sel_c.size == 0:
            continue
        g = torch.from_numpy(gid_need[sel_c])
        at = torch.from_numpy(sel_c)
        proj = projection_ref(means[g].to(dtype), None, quats[g].to(dtype),
                              scales[g].to(dtype), viewmats[c:c + 1].to(dtype),
                              Ks[c:c + 1].to(dtype), width, height, eps2d, near_plane,
                              far_plane, radius_clip, calc_comp, camera_model,
                              opacities[g].to(dtype))
        m2_rows = m2_rows.index_copy(0, at, proj["means2d"][0])
        con_rows = con_rows.index_copy(0, at, proj["conics"][0])
        dep_rows = dep_rows.index_copy(0, at, proj["depths"][0])
        if calc_comp:
            comp_rows = comp_rows.index_copy(0, at, proj["compensations"][0])
        if sh_degree is not None:
            dirs = means[g].to(dtype) - campos[c][None, :]
            f = spherical_harmonics_ref(sh_degree, dirs, colors[g].to(dtype))
            f = torch.clamp_min(f + 0.5, 0.0)
        else:
            f = colors[g].to(dtype)
        feat_parts.append((at, f))
    op_rows = opacities.to(dtype)[torch.from_numpy(gid_need)]
    if calc_comp:
        op_rows = op_rows * comp_rows
    Dc = colors.shape[-1]
    feats = torch.zeros(n_need, Dc, dtype=dtype)
    for at, f in feat_parts:
        feats = feats.index_copy(0, at, f)
    if render_mode in ("D", "ED"):
        feats = dep_rows[:, None]
    elif render_mode in ("RGB+D", "RGB+ED"):
        feats = torch.cat([feats, dep_rows[:, None]], dim=-1)
    bg = backgrounds.to(dtype) if backgrounds is not None else None
    if bg is not None and render_mode in ("RGB+D", "RGB+ED"):
        bg = torch.cat([bg, torch.zeros(C, 1, dtype=dtype)], dim=-1)
    elif bg is not None and render_mode in ("D", "ED"):
        bg = torch.zeros(C, 1, dtype=dtype)
    fr = flat_need
    dec = {"means2d": ex_m2[fr], "conics": ex_con[fr], "opacities": ex_op[fr]}
    rc, ra, info = rasterize_to_pixels_ref(
        m2_rows, con_rows, feats, op_rows, width, height, tile_size,
        torch.from_numpy(offsets), torch.from_numpy(np.ascontiguousarray(fl)),
        backgrounds=bg, masks=masks, decide=dec, dtype=dtype)
    if render_mode in ("ED", "RGB+ED"):
        rc = torch.cat([rc[..., :-1], rc[..., -1:] / ra.clamp(min=1e-10)], dim=-1)
    meta = {"isect_ids": isect_ids, "flatten_ids": flatten_ids, "offsets": offsets,
            "valid": ex["valid"], "radii": ex["radii"],
            "transmittance": info["transmittance"],
            "last_ids": info["last_ids"], "n_isects": int(isect_ids.shape[0])}
    return rc, ra, meta


def grad2d_stats_ref(grads, gaussian_ids, radii, n_gaussians, width, height,
                     n_cameras, grad2d=None, count=None):
    """Densification statistics of DefaultStrategy._update_state
    (gsplat/strategy/default.py:235-268), in float64 on the host.

    grads [nnz, 2] with ``gaussian_ids`` [nnz] (packed), or grads [..., N, 2]
    with ``radii`` [..., N, 2] (dense; rows count where both radii are > 0).
    Adds ||grads * (W/2 * C, H/2 * C)|| and 1 per visible row to the
    Gaussian's accumulators; returns (grad2d, count)."""
    g = grads.detach().double().clone()
    g[..., 0] *= width / 2.0 * n_cameras
    g[..., 1] *= height / 2.0 * n_cameras
    if gaussian_ids is None:
        sel = (radii > 0).all(dim=-1)
        ids = torch.where(sel)[-1]
        g = g[sel]
    else:
        ids = gaussian_ids
    out_g = torch.zeros(n_gaussians, dtype=torch.float64) if grad2d is None \
        else grad2d.double().clone()
    out_c = torch.zeros(n_gaussians, dtype=torch.float64) if count is None \
        else count.double().clone()
    out_g.index_add_(0, ids, g.norm(dim=-1))
    out_c.index_add_(0, ids, torch.ones(ids.shape[0], dtype=torch.float64))
    return out_g, out_c
