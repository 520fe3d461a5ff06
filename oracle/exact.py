"""Bit-exact host oracle (TEST INFRASTRUCTURE ONLY).

numpy front end of ``exact_ref.c`` plus the integer logic that is clearer in
numpy.  Each function cites the reference code it restates.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path
from typing import Optional, Tuple

import numpy as np

_HERE = Path(__file__).resolve().parent
_SO = _HERE / "build" / "liboracle.so"
_lib = None

ALPHA_THRESHOLD = np.float32(1.0) / np.float32(255.0)
MAX_ALPHA = np.float32(0.99)
TRANSMITTANCE_THRESHOLD = np.float32(1e-4)


def build() -> Path:
    """Compile exact_ref.c with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _SO


def _load():
    global _lib
    if _lib is None:
        if not _SO.exists():
            build()
        _lib = ctypes.CDLL(str(_SO))
    return _lib


def _p(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> Optional[np.ndarray]:
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


# --------------------------------------------------------------------------
# log
# --------------------------------------------------------------------------
_LN2_HI = np.float32(float.fromhex("0x1.62e3p-1"))
_LN2_LO = np.float32(float.fromhex("0x1.2fefa2p-17"))
_SQRT2 = np.float32(1.41421356)
_C1, _C2, _C3, _C4 = (np.float32(0.666666667), np.float32(0.4),
                      np.float32(0.285714286), np.float32(0.222222222))


def portable_logf(x) -> np.ndarray:
    """numpy float32 restatement of the device ``portable_logf`` (every op a
    single IEEE float32 operation, same order), so results are bit-identical
    to the GPU and to ``oracle_portable_logf`` in exact_ref.c."""
    x = np.array(x, dtype=np.float32, copy=True, ndmin=1)
    bits = x.view(np.uint32)
    e = ((bits >> np.uint32(23)) & np.uint32(0xFF)).astype(np.int32) - 127
    m = ((bits & np.uint32(0x7FFFFF)) | np.uint32(0x3F800000)).view(np.float32).copy()
    sub = e == -127
    if np.any(sub):
        xs = x[sub] * np.float32(8388608.0)
        b2 = xs.view(np.uint32)
        e[sub] = ((b2 >> np.uint32(23)) & np.uint32(0xFF)).astype(np.int32) - 127 - 23
        m[sub] = ((b2 & np.uint32(0x7FFFFF)) | np.uint32(0x3F800000)).view(np.float32)
    big = m > _SQRT2
    m = np.where(big, m * np.float32(0.5), m).astype(np.float32)
    e = e + big.astype(np.int32)
    f = m - np.float32(1.0)
    s = f / (np.float32(2.0) + f)
    z = s * s
    r = z * (_C1 + z * (_C2 + z * (_C3 + z * _C4)))
    lnm = (s + s) + s * r
    ef = e.astype(np.float32)
    out = (ef * _LN2_HI + (lnm + ef * _LN2_LO)).astype(np.float32)
    with np.errstate(invalid="ignore"):
        out[~(x > 0)] = np.float32(np.nan)
    out[x == np.float32(np.inf)] = np.float32(np.inf)
    return out


def portable_logf_c(x) -> np.ndarray:
    """Same function through the C oracle (used to cross-check the numpy one)."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    y = np.empty_like(x)
    _load().oracle_portable_logf_array(_p(x), _p(y), ctypes.c_int64(x.size))
    return y


def portable_expf(x) -> np.ndarray:
    """e^x exactly as the device ``portable_expf`` computes it (through the C
    oracle, whose fmaf/rintf give the same correctly rounded operations);
    the rasterizer's alpha is o * portable_expf(-sigma)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    flat = x.ravel()
    y = np.empty_like(flat)
    _load().oracle_portable_expf_array(_p(flat), _p(y), ctypes.c_int64(flat.size))
    return y.reshape(x.shape)


# --------------------------------------------------------------------------
# Projection (ProjectionEWA3DGSFused.cu:38-234)
# --------------------------------------------------------------------------
def projection_fwd(means, covars, quats, scales, opacities, viewmats, Ks, width,
                   height, eps2d=0.3, near_plane=0.01, far_plane=1e10,
                   radius_clip=0.0, calc_compensations=False, camera_model=0):
    """Dense projection of the [..., C, N] rows.  Returns a dict of numpy
    arrays: radii (int32), means2d, depths, conics, compensations (or None) and
    valid (bool)."""
    means = _f32(means)
    batch_dims = means.shape[:-2]
    N = means.shape[-2]
    C = viewmats.shape[-3]
    B = int(np.prod(batch_dims)) if batch_dims else 1
    covars, quats, scales, opacities = map(_f32, (covars, quats, scales, opacities))
    viewmats, Ks = _f32(viewmats), _f32(Ks)
    rows = B * C * N
    radii = np.zeros((rows, 2), np.int32)
    means2d = np.zeros((rows, 2), np.float32)
    depths = np.zeros(rows, np.float32)
    conics = np.zeros((rows, 3), np.float32)
    comps = np.zeros(rows, np.float32) if calc_compensations else None
    valid = np.zeros(rows, np.uint8)
    lib = _load()
    lib.oracle_projection_fwd(
        ctypes.c_int64(B), ctypes.c_int64(C), ctypes.c_int64(N), _p(means),
        _p(covars), _p(quats), _p(scales), _p(opacities), _p(viewmats), _p(Ks),
        ctypes.c_int32(width), ctypes.c_int32(height), ctypes.c_float(eps2d),
        ctypes.c_float(near_plane), ctypes.c_float(far_plane),
        ctypes.c_float(radius_clip), ctypes.c_int32(int(calc_compensations)),
        ctypes.c_int32(camera_model), _p(radii), _p(means2d), _p(depths),
        _p(conics), _p(comps), _p(valid))
    shp = tuple(batch_dims) + (C, N)
    return {
        "radii": radii.reshape(shp + (2,)),
        "means2d": means2d.reshape(shp + (2,)),
        "depths": depths.reshape(shp),
        "conics": conics.reshape(shp + (3,)),
        "compensations": None if comps is None else comps.reshape(shp),
        "valid": valid.reshape(shp).astype(bool),
    }


def pack_projection(dense: dict, B: int, C: int, N: int) -> dict:
    """Packed layout of a dense projection (ProjectionEWA3DGSPacked.cu:248-284):
    valid rows in (b, c, g) row-major order + CSR indptr over the B*C rows."""
    valid = dense["valid"].reshape(B * C * N)
    rows = np.nonzero(valid)[0]
    bc, g = rows // N, rows % N
    counts = valid.reshape(B * C, N).sum(axis=1)
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    out = {
        "indptr": indptr,
        "batch_ids": (bc // C).astype(np.int64),
        "camera_ids": (bc % C).astype(np.int64),
        "gaussian_ids": g.astype(np.int64),
    }
    for k in ("radii", "means2d", "depths", "conics", "compensations"):
        v = dense[k]
        if v is None:
            out[k] = None
            continue
        v = v.reshape((B * C * N,) + v.shape[len(dense["valid"].shape):])
        out[k] = v[rows]
    return out


# --------------------------------------------------------------------------
# Tile intersection (IntersectTile.cu:133-288, Intersect.cpp:33-164)
# --------------------------------------------------------------------------
def isect_tiles(means2d, radii, depths, tile_size, tile_width, tile_height,
                sort=True, packed=False, n_images=None, image_ids=None,
                conics=None, opacities=None):
    """Returns (tiles_per_gauss int32, isect_ids int64, flatten_ids int32).

    Sorted order: keys ascending, ties in emission (row) order -- the stable
    radix sort of the reference (IntersectTile.cu:496-505)."""
    means2d = _f32(means2d)
    radii = np.ascontiguousarray(radii, dtype=np.int32)
    depths = _f32(depths)
    conics = _f32(conics)
    opacities = _f32(opacities)
    if packed:
        n = means2d.shape[0]
        N = 0
        I = int(n_images)
        image_ids = np.ascontiguousarray(image_ids, dtype=np.int64)
    else:
        N = means2d.shape[-2]
        I = int(np.prod(means2d.shape[:-2])) if means2d.ndim > 2 else 1
        n = I * N
        image_ids = None
    tile_n_bits = int(tile_width * tile_height).bit_length()
    lib = _load()
    counts = np.zeros(n, np.int32)
    mf, rf = means2d.reshape(n, 2), radii.reshape(n, 2)
    cf = conics.reshape(n, 3) if conics is not None else None
    of = opacities.reshape(n) if opacities is not None else None
    lib.oracle_isect_count(ctypes.c_int64(n), _p(mf), _p(rf), _p(cf), _p(of),
                           ctypes.c_int32(tile_size), ctypes.c_int32(tile_width),
                           ctypes.c_int32(tile_height), _p(counts))
    cum = np.cumsum(counts.astype(np.int64))
    n_isects = int(cum[-1]) if n else 0
    row_off = np.ascontiguousarray(cum - counts)
    isect_ids = np.zeros(n_isects, np.int64)
    flatten_ids = np.zeros(n_isects, np.int32)
    scratch = np.zeros(max(int(counts.max()) if n else 0, 1), np.int64)
    if n_isects:
        lib.oracle_isect_emit(
            ctypes.c_int64(n), ctypes.c_int64(max(N, 1)), _p(image_ids), _p(mf),
            _p(rf), _p(depths.reshape(n)), _p(cf), _p(of), ctypes.c_int32(tile_size),
            ctypes.c_int32(tile_width), ctypes.c_int32(tile_height),
            ctypes.c_int32(tile_n_bits), _p(row_off), _p(scratch), _p(isect_ids),
            _p(flatten_ids))
    if sort and n_isects:
        order = np.argsort(isect_ids, kind="stable")
        isect_ids, flatten_ids = isect_ids[order], flatten_ids[order]
    tiles_shape = depths.shape
    return counts.reshape(tiles_shape), isect_ids, flatten_ids


def isect_tiles_box_python(means2d, radii, depths, tile_size, tile_width, tile_height):
    """Pure-Python loop restatement of the reference's own torch oracle
    ``_isect_tiles`` (gsplat/cuda/_torch_impl.py:344-439), box test, unsorted
    rows then sorted -- for small inputs only."""
    means2d = np.asarray(means2d, np.float32)
    radii = np.asarray(radii, np.int32)
    depths = np.asarray(depths, np.float32)
    image_dims = means2d.shape[:-2]
    N = means2d.shape[-2]
    I = int(np.prod(image_dims)) if image_dims else 1
    m = means2d.reshape(I, N, 2)
    r = radii.reshape(I, N, 2)
    d = depths.reshape(I, N)
    ts = np.float32(tile_size)
    tile_n_bits = int(tile_width * tile_height).bit_length()
    keys, flat, counts = [], [], np.zeros((I, N), np.int32)
    for i in range(I):
        for g in range(N):
            if r[i, g, 0] <= 0 or r[i, g, 1] <= 0:
                continue
            tx, ty = m[i, g, 0] / ts, m[i, g, 1] / ts
            rx, ry = np.float32(r[i, g, 0]) / ts, np.float32(r[i, g, 1]) / ts
            x0 = min(max(0, int(np.floor(tx - rx))), tile_width)
            y0 = min(max(0, int(np.floor(ty - ry))), tile_height)
            x1 = min(max(0, int(np.ceil(tx + rx))), tile_width)
            y1 = min(max(0, int(np.ceil(ty + ry))), tile_height)
            counts[i, g] = (x1 - x0) * (y1 - y0)
            dbits = int(np.float32(d[i, g]).view(np.uint32))
            for y in range(y0, y1):
                for x in range(x0, x1):
                    keys.append((i << (32 + tile_n_bits)) | ((y * tile_width + x) << 32) | dbits)
                    flat.append(i * N + g)
    keys = np.array(keys, np.int64)
    flat = np.array(flat, np.int32)
    order = np.argsort(keys, kind="stable")
    return counts.reshape(image_dims + (N,)), keys[order], flat[order]


def isect_offset_encode(isect_ids, n_images, tile_width, tile_height) -> np.ndarray:
    """offsets[i, t] = #{k : isect_ids[k] >> 32 < (i << tile_n_bits | t)}
    (gsplat/cuda/_torch_impl.py:443-469, IntersectTile.cu:391-474)."""
    n_tiles = tile_width * tile_height
    tile_n_bits = int(n_tiles).bit_length()
    hi = np.asarray(isect_ids, np.int64) >> 32
    img = np.arange(n_images, dtype=np.int64)[:, None]
    tid = np.arange(n_tiles, dtype=np.int64)[None, :]
    q = (img << tile_n_bits) | tid
    offs = np.searchsorted(hi, q.ravel(), side="left").astype(np.int32)
    return offs.reshape(n_images, tile_height, tile_width)


# --------------------------------------------------------------------------
# Adam (AdamCUDA.cu:56-68)
# --------------------------------------------------------------------------
def adam(param, grad, exp_avg, exp_avg_sq, valid, lr, b1, b2, eps):
    """One step, float32, the kernel's operation order.  Returns new
    (param, exp_avg, exp_avg_sq); rows with valid == False are unchanged."""
    p = np.array(param, np.float32, copy=True)
    g = np.asarray(grad, np.float32)
    m = np.array(exp_avg, np.float32, copy=True)
    v = np.array(exp_avg_sq, np.float32, copy=True)
    b1, b2, lr, eps = (np.float32(x) for x in (b1, b2, lr, eps))
    one = np.float32(1.0)
    m_new = b1 * m + (one - b1) * g
    v_new = b2 * v + (one - b2) * g * g
    step = -lr * m_new / (np.sqrt(v_new) + eps)
    p_new = p + step
    if valid is not None:
        sel = np.asarray(valid, bool).reshape((-1,) + (1,) * (p.ndim - 1))
        sel = np.broadcast_to(sel, p.shape)
        p_new = np.where(sel, p_new, p)
        m_new = np.where(sel, m_new, m)
        v_new = np.where(sel, v_new, v)
    return p_new.astype(np.float32), m_new.astype(np.float32), v_new.astype(np.float32)


# --------------------------------------------------------------------------
# Rasterizer decisions (RasterizeToPixels3DGSFwd.cu:165-194)
# --------------------------------------------------------------------------
def gauss_sigma_f32(a, b, c, dx, dy) -> np.ndarray:
    """0.5 * ((a dx) dx + (c dy) dy) + (b dx) dy in float32, uncontracted."""
    a, b, c, dx, dy = (np.asarray(v, np.float32) for v in (a, b, c, dx, dy))
    half = np.float32(0.5)
    return (half * ((a * dx) * dx + (c * dy) * dy) + (b * dx) * dy).astype(np.float32)


def alpha_thresholds(opacity) -> Tuple[np.ndarray, np.ndarray]:
    """(sig_max, sig_clamp): a Gaussian composites at sigma iff
    0 <= sigma <= sig_max, and its alpha is clamped to 0.99 iff sigma <
    sig_clamp (alpha < 1/255 <=> sigma > ln(o*255), o e^-sigma > 0.99 <=>
    sigma < ln(o/0.99))."""
    o = np.asarray(opacity, np.float32)
    pos = o > 0
    with np.errstate(divide="ignore", invalid="ignore"):
        sig_max = np.where(pos, portable_logf(o / ALPHA_THRESHOLD).reshape(o.shape),
                           np.float32(-np.inf))
        sig_clamp = np.where(pos, portable_logf(o / MAX_ALPHA).reshape(o.shape),
                             np.float32(-np.inf))
    return sig_max.astype(np.float32), sig_clamp.astype(np.float32)


# --------------------------------------------------------------------------
# Rasterize to indices (RasterizeToIndices3DGS.cu:36-196, both passes;
# Rasterization.cpp:216-308)
# --------------------------------------------------------------------------
def rasterize_to_indices(range_start, range_end, transmittances, means2d, conics,
                         opacities, width, height, tile_size, tile_offsets,
                         flatten_ids, N):
    """The (gaussian, pixel) pairs a pixel composites over the isect batches
    [range_start, range_end) of its tile (batches of tile_size^2), starting
    from its given transmittance; pixel-major order, depth order within a
    pixel.  Decisions are the device's: float32 sigma in the kernels' order,
    thresholds from ``alpha_thresholds``, alpha = o * portable_expf(-sigma)
    clamped at 0.99, stop (exclusive) once T (1 - alpha) <= 1e-4.  A plain
    per-pixel loop: for small inputs only.  Returns int64 arrays
    (gaussian_ids = row % N, pixel_ids = image * H * W + i * W + j)."""
    offs = np.asarray(tile_offsets, np.int64)
    th, tw = offs.shape[-2:]
    offs = offs.reshape(-1)
    I = offs.size // (th * tw)
    fids = np.asarray(flatten_ids, np.int64)
    n_isects = fids.size
    xy = np.asarray(means2d, np.float32).reshape(-1, 2)
    con = np.asarray(conics, np.float32).reshape(-1, 3)
    op = np.asarray(opacities, np.float32).reshape(-1)
    sig_max, sig_clamp = alpha_thresholds(op)
    T0 = np.asarray(transmittances, np.float32).reshape(-1)
    bs = tile_size * tile_size
    out_g, out_p = [], []
    for img in range(I):
        for i in range(height):
            for j in range(width):
                tile = (i // tile_size) * tw + j // tile_size
                slot = img * th * tw + tile
                s = offs[slot]
                e = n_isects if slot == I * th * tw - 1 else offs[slot + 1]
                n_batches = (e - s + bs - 1) // bs
                pix = (img * height + i) * width + j
                T = np.float32(T0[pix])
                px, py = np.float32(j + 0.5), np.float32(i + 0.5)
                stop = False
                for b in range(range_start, min(range_end, n_batches)):
                    for k in range(s + b * bs, min(s + (b + 1) * bs, e)):
                        g = fids[k]
                        sig = gauss_sigma_f32(con[g, 0], con[g, 1], con[g, 2],
                                              xy[g, 0] - px, xy[g, 1] - py)
                        if sig < 0 or not (sig <= sig_max[g]):
                            continue
                        if sig < sig_clamp[g]:
                            alpha = MAX_ALPHA
                        else:
                            alpha = np.float32(op[g] * portable_expf(-sig).reshape(()))
                        nxt = np.float32(T * np.float32(np.float32(1.0) - alpha))
                        if nxt <= TRANSMITTANCE_THRESHOLD:
                            stop = True
                            break
                        out_g.append(g % N)
                        out_p.append(pix)
                        T = nxt
                    if stop:
                        break
    return np.asarray(out_g, np.int64), np.asarray(out_p, np.int64)
