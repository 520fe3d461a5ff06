"""Shared helpers for the parity tests."""

import math

import numpy as np
import torch

from gsplat_amd._helper import look_at_viewmat
from oracle import exact

DEV = "cuda:0"


def small_scene(seed=0, N=2000, C=2, W=160, H=120, f=150.0, opac_range=(0.05, 1.0),
                scale_range=(0.01, 0.12), spread=1.2):
    """Random 3D Gaussians in front of C cameras (CPU float32 tensors)."""
    g = torch.Generator().manual_seed(seed)
    means = torch.randn(N, 3, generator=g) * spread
    quats = torch.randn(N, 4, generator=g)
    scales = torch.rand(N, 3, generator=g) * (scale_range[1] - scale_range[0]) + scale_range[0]
    opac = torch.rand(N, generator=g) * (opac_range[1] - opac_range[0]) + opac_range[0]
    vms = [look_at_viewmat((4 * math.sin(0.5 * k), -0.5, -4 * math.cos(0.5 * k)))
           for k in range(C)]
    vm = torch.stack(vms)
    K = torch.tensor([[f, 0, W / 2], [0, f, H / 2], [0, 0, 1]]).expand(C, 3, 3).contiguous()
    return means, quats, scales, opac, vm, K, W, H


def projected_2d(seed=0, N=2000, C=2, W=160, H=120, tile=16, D=3, packed=False,
                 **scene_kw):
    """Exact-oracle projection + intersection of a random scene: the float32
    inputs of the rasterizer and its tile lists (numpy/torch CPU).
    ``scene_kw`` goes to small_scene (opacity and scale ranges, spread)."""
    means, quats, scales, opac, vm, K, W, H = small_scene(seed, N, C, W, H, **scene_kw)
    ex = exact.projection_fwd(means.numpy(), None, quats.numpy(), scales.numpy(),
                              opac.numpy(), vm.numpy(), K.numpy(), W, H)
    g = torch.Generator().manual_seed(seed + 1)
    colors = torch.rand(C, N, D, generator=g)
    ops = np.broadcast_to(opac.numpy()[None], (C, N)).copy()
    tw, th = math.ceil(W / tile), math.ceil(H / tile)
    if packed:
        valid = ex["valid"].reshape(-1)
        rows = np.nonzero(valid)[0]
        m2 = ex["means2d"].reshape(-1, 2)[rows]
        con = ex["conics"].reshape(-1, 3)[rows]
        dep = ex["depths"].reshape(-1)[rows]
        rad = ex["radii"].reshape(-1, 2)[rows]
        op = ops.reshape(-1)[rows]
        col = colors.reshape(-1, D)[rows]
        image_ids = (rows // N).astype(np.int64)
        tpg, ids, fl = exact.isect_tiles(m2, rad, dep, tile, tw, th, packed=True,
                                         n_images=C, image_ids=image_ids,
                                         conics=con, opacities=op)
    else:
        m2, con, dep, rad, op, col = (ex["means2d"], ex["conics"], ex["depths"],
                                      ex["radii"], ops, colors)
        tpg, ids, fl = exact.isect_tiles(m2, rad, dep, tile, tw, th, conics=con,
                                         opacities=op)
    offs = exact.isect_offset_encode(ids, C, tw, th)
    return {
        "means2d": torch.from_numpy(np.ascontiguousarray(m2)),
        "conics": torch.from_numpy(np.ascontiguousarray(con)),
        "opacities": torch.from_numpy(np.ascontiguousarray(op)),
        "colors": col.contiguous(),
        "offsets": torch.from_numpy(offs),
        "flatten_ids": torch.from_numpy(fl),
        "W": W, "H": H, "tile": tile, "C": C,
    }


def report(a, b, name):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    d = (a - b).abs()
    rel = d / b.abs().clamp(min=1e-12)
    return (f"{name}: max abs {d.max().item():.3e}, max rel {rel.max().item():.3e}, "
            f"numel {a.numel()}")


def assert_close(a, b, rtol, atol, name):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    ok = (a - b).abs() <= atol + rtol * b.abs()
    if not bool(ok.all()):
        bad = (~ok).sum().item()
        raise AssertionError(f"{report(a, b, name)}; {bad} elements outside "
                             f"rtol={rtol} atol={atol}")


GRAD_STRICT_SLACK = 5e-4  # strict-tolerance pass rate may trail fp32's by this
GRAD_MAX_RATIO = 2.0      # worst element may exceed fp32's worst by this factor
GRAD_RMS_RATIO = 1.5      # RMS error may exceed fp32's by this factor


def assert_grad_close(got, ref64, ref32, rtol, atol, name):
    """Gradient parity at the float32 floor.

    ``ref64`` is the float64 restatement (the exact value of the algorithm),
    ``ref32`` the same restatement evaluated in float32 -- what any float32
    implementation of the reference's PyTorch path computes.  Where a
    gradient is a sum of many cancelling per-pixel or per-camera terms,
    float32 cannot reach rtol/atol against the exact value (``ref32`` itself
    misses it on a fraction of elements), and two float32 evaluations round
    such elements independently.  So the comparison is statistical, against
    the float32 restatement's own error |ref32 - ref64|:

      * the fraction of elements within tol = atol + rtol |ref64| may trail
        the float32 restatement's by at most 0.05 percentage points;
      * measured in units of tol, the RMS deviation from ref64 may be at
        most max(1, 1.5x) the float32 restatement's and the largest at most
        max(1, 2x): the worst elements are sums whose terms cancel by two
        to three orders of magnitude, and two float32 summation orders of the
        same terms land up to ~2x apart on them;
      * where the float32 restatement holds rtol/atol on every element, the
        gradient must too (the elementwise tolerance as a hard gate).

    Returns the report line."""
    a = got.detach().double().cpu()
    r = ref64.detach().double().cpu()
    r32 = ref32.detach().double().cpu()
    assert a.shape == r.shape == r32.shape, (name, a.shape, r.shape, r32.shape)
    assert bool(torch.isfinite(a).all()), f"{name}: non-finite values"
    err = (a - r).abs()
    err32 = (r32 - r).abs()
    tol = atol + rtol * r.abs()
    e, e32 = err / tol, err32 / tol
    frac = (e <= 1).double().mean().item()
    frac32 = (e32 <= 1).double().mean().item()
    mx, mx32 = e.max().item(), e32.max().item()
    rms, rms32 = e.square().mean().sqrt().item(), e32.square().mean().sqrt().item()
    worst = int(e.reshape(-1).argmax())
    msg = (f"{name}: numel {err.numel()}; within rtol={rtol} atol={atol}: {frac:.5f} "
           f"(fp32 restatement {frac32:.5f}); in units of tol: max {mx:.3g} "
           f"(fp32 {mx32:.3g}), rms {rms:.3g} (fp32 {rms32:.3g}); max abs "
           f"{err.max().item():.3e} (fp32 {err32.max().item():.3e}); worst element "
           f"{worst}: got {a.reshape(-1)[worst].item():.9g}, float64 "
           f"{r.reshape(-1)[worst].item():.9g}, float32 {r32.reshape(-1)[worst].item():.9g}")
    print("[grad gate]", msg)  # shown with pytest -rP
    assert frac >= frac32 - GRAD_STRICT_SLACK, msg
    if frac32 == 1.0:
        assert frac == 1.0, "elementwise tolerance (float32 holds it): " + msg
    assert mx <= max(1.0, GRAD_MAX_RATIO * mx32), msg
    assert rms <= max(1.0, GRAD_RMS_RATIO * rms32), msg
    return msg
