"""Tile rasterizer on the GPU against the PyTorch restatement
(gsplat/cuda/_torch_impl.py:472-683, compositing rules of
RasterizeToPixels3DGSFwd.cu:140-212); backward against autograd.
Reference test: tests/test_basic.py:1954-2063.

The compositing decisions (which Gaussians each pixel takes, where it
stops) are restated bit for bit -- alpha is o * portable_expf(-sigma) on
both sides -- so last_ids and the final transmittance (render_alphas =
1 - T) must match exactly on every pixel.  Renders must match the float64
restatement within rtol 1e-4 / atol 1e-5; gradients are held to that
tolerance at the float32 floor (tests/_util.py:assert_grad_close), using the
same restatement evaluated in float32 as the measure of that floor."""

import math

import numpy as np
import pytest
import torch

from oracle import torch_ref
from tests._util import DEV, assert_close, assert_grad_close, projected_2d

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-5


def _run(data, packed, D, backgrounds, masks, absgrad=False):
    from gsplat_amd.cuda._wrapper import rasterize_to_pixels
    W, H, ts, C = data["W"], data["H"], data["tile"], data["C"]
    m2, con, op, col = data["means2d"], data["conics"], data["opacities"], data["colors"]
    offs, fl = data["offsets"], data["flatten_ids"]
    g = torch.Generator().manual_seed(11)
    bg = torch.rand(C, D, generator=g) if backgrounds else None
    mk = (torch.rand(offs.shape, generator=g) > 0.2) if masks else None
    v_rc = torch.randn(C, H, W, D, generator=g)
    v_ra = torch.randn(C, H, W, 1, generator=g)

    # oracle forward (float64)
    ins_ref = [t.double().requires_grad_() for t in (m2, con, col, op)]
    bg_ref = bg.double().requires_grad_() if bg is not None else None
    rc_r, ra_r, info = torch_ref.rasterize_to_pixels_ref(
        ins_ref[0], ins_ref[1], ins_ref[2], ins_ref[3], W, H, ts, offs, fl,
        backgrounds=bg_ref, masks=mk)
    ((rc_r * v_rc.double()).sum() + (ra_r * v_ra.double()).sum()).backward()
    # the same restatement in float32 (its error measures the fp32 floor)
    ins32 = [t.float().clone().requires_grad_() for t in (m2, con, col, op)]
    bg32 = bg.float().clone().requires_grad_() if bg is not None else None
    rc32, ra32, _ = torch_ref.rasterize_to_pixels_ref(
        ins32[0], ins32[1], ins32[2], ins32[3], W, H, ts, offs, fl,
        backgrounds=bg32, masks=mk, dtype=torch.float32)
    ((rc32 * v_rc).sum() + (ra32 * v_ra).sum()).backward()

    ins = [t.clone().to(DEV).requires_grad_() for t in (m2, con, col, op)]
    bgd = bg.clone().to(DEV).requires_grad_() if bg is not None else None
    rc, ra = rasterize_to_pixels(ins[0], ins[1], ins[2], ins[3], W, H, ts, offs.to(DEV),
                                 fl.to(DEV), backgrounds=bgd,
                                 masks=mk.to(DEV) if mk is not None else None,
                                 packed=packed, absgrad=absgrad)
    ((rc * v_rc.to(DEV)).sum() + (ra * v_ra.to(DEV)).sum()).backward()

    # decisions are exact: alpha = 1 - T with T the float32 running product
    alpha32 = (np.float32(1.0) - info["transmittance"]).astype(np.float32)
    np.testing.assert_array_equal(ra.detach().cpu().numpy()[..., 0], alpha32)
    assert_close(rc.cpu(), rc_r.detach(), RTOL, ATOL, "render_colors")
    assert_close(ra.cpu(), ra_r.detach(), RTOL, ATOL, "render_alphas")
    for name, a, b, b32 in zip(("v_means2d", "v_conics", "v_colors", "v_opacities"),
                               ins, ins_ref, ins32):
        assert_grad_close(a.grad, b.grad, b32.grad, RTOL, ATOL, name)
    if bg is not None:
        assert_grad_close(bgd.grad, bg_ref.grad, bg32.grad, RTOL, ATOL, "v_backgrounds")
    return ins


@pytest.mark.parametrize("D", [1, 3, 4, 8, 17, 32])
@pytest.mark.parametrize("packed", [False, True])
def test_rasterize_fwd_bwd(D, packed):
    data = projected_2d(seed=D, N=3000, C=2, D=D, packed=packed)
    _run(data, packed, D, backgrounds=False, masks=False)


def test_rasterize_backgrounds_and_masks():
    data = projected_2d(seed=21, N=3000, C=2, D=3)
    _run(data, False, 3, backgrounds=True, masks=True)


@pytest.mark.parametrize("tile", [8, 16])
def test_rasterize_tile_sizes(tile):
    data = projected_2d(seed=22, N=2000, C=1, D=3, tile=tile)
    _run(data, False, 3, backgrounds=True, masks=False)


def test_rasterize_padded_and_chunked_channels():
    # 6 channels pad to 8; 40 channels run as 32 + 8
    for D in (6, 40):
        data = projected_2d(seed=30 + D, N=1500, C=1, D=D)
        _run(data, False, D, backgrounds=True, masks=False)


def test_rasterize_absgrad_is_sum_of_abs():
    """absgrad = sum over pixels of |dL/dmean2d| (RasterizeToPixels3DGSBwd.cu:256-258):
    equal to the plain gradient when a single pixel has nonzero upstream grad."""
    from gsplat_amd.cuda._wrapper import rasterize_to_pixels
    data = projected_2d(seed=40, N=1000, C=1, D=3)
    W, H, ts = data["W"], data["H"], data["tile"]
    m2 = data["means2d"].clone().to(DEV).requires_grad_()
    rc, ra = rasterize_to_pixels(m2, data["conics"].to(DEV), data["colors"].to(DEV),
                                 data["opacities"].to(DEV), W, H, ts,
                                 data["offsets"].to(DEV), data["flatten_ids"].to(DEV),
                                 absgrad=True)
    w = torch.zeros_like(rc)
    w[0, 60, 80] = 1.0
    (rc * w).sum().backward()
    torch.testing.assert_close(m2.absgrad, m2.grad.abs(), rtol=1e-6, atol=1e-8)
    # and it upper-bounds |grad| for a dense upstream gradient
    m2b = data["means2d"].clone().to(DEV).requires_grad_()
    rc, ra = rasterize_to_pixels(m2b, data["conics"].to(DEV), data["colors"].to(DEV),
                                 data["opacities"].to(DEV), W, H, ts,
                                 data["offsets"].to(DEV), data["flatten_ids"].to(DEV),
                                 absgrad=True)
    (rc * torch.randn_like(rc)).sum().backward()
    assert bool((m2b.absgrad + 1e-6 >= m2b.grad.abs()).all())


def test_rasterize_last_ids_match_oracle():
    from gsplat_amd.cuda import _ops
    data = projected_2d(seed=50, N=3000, C=2, D=3)
    W, H, ts = data["W"], data["H"], data["tile"]
    _, _, info = torch_ref.rasterize_to_pixels_ref(
        data["means2d"].double(), data["conics"].double(), data["colors"].double(),
        data["opacities"].double(), W, H, ts, data["offsets"], data["flatten_ids"])
    rc, ra, last = _ops.rasterize_to_pixels_3dgs_fwd(
        data["means2d"].to(DEV), data["conics"].to(DEV), data["colors"].to(DEV),
        data["opacities"].to(DEV), None, None, W, H, ts, data["offsets"].to(DEV),
        data["flatten_ids"].to(DEV))
    np.testing.assert_array_equal(last.cpu().numpy(), info["last_ids"])
    np.testing.assert_array_equal(ra.cpu().numpy()[..., 0],
                                  (np.float32(1.0) - info["transmittance"]).astype(np.float32))


@pytest.mark.parametrize("D,bg,packed", [(4, False, True), (4, True, False), (1, False, True)])
def test_rasterize_expected_depth_in_kernel(D, bg, packed):
    """The expected-depth channel divided by max(alpha, 1e-10) inside the
    rasterizer (render modes RGB+ED and ED) against the reference's torch
    form of it (rendering.py:1259-1267) applied to the float64 and float32
    restatements: render within rtol/atol, gradients through the gate, and
    the render bit for bit equal to the same division by torch of the plain
    kernel's output."""
    from gsplat_amd.cuda._wrapper import _rasterize_to_pixels, rasterize_to_pixels
    data = projected_2d(seed=70 + D, N=2000, C=2, D=D, packed=packed)
    W, H, ts, C = data["W"], data["H"], data["tile"], data["C"]
    m2, con, op, col = data["means2d"], data["conics"], data["opacities"], data["colors"]
    offs, fl = data["offsets"], data["flatten_ids"]
    g = torch.Generator().manual_seed(12)
    bgt = torch.rand(C, D, generator=g) if bg else None
    v_rc = torch.randn(C, H, W, D, generator=g)
    v_ra = torch.randn(C, H, W, 1, generator=g)

    def ed(rc, ra):
        return torch.cat([rc[..., :-1], rc[..., -1:] / ra.clamp(min=1e-10)], dim=-1)

    outs = {}
    for name, dtype in (("64", torch.float64), ("32", torch.float32)):
        ins = [t.to(dtype).clone().requires_grad_() for t in (m2, con, col, op)]
        bgr = bgt.to(dtype).clone().requires_grad_() if bg else None
        rc, ra, _ = torch_ref.rasterize_to_pixels_ref(
            ins[0], ins[1], ins[2], ins[3], W, H, ts, offs, fl,
            backgrounds=bgr, dtype=dtype)
        rc = ed(rc, ra)
        ((rc * v_rc.to(dtype)).sum() + (ra * v_ra.to(dtype)).sum()).backward()
        outs[name] = (rc.detach(), ins, bgr)
    ins = [t.clone().to(DEV).requires_grad_() for t in (m2, con, col, op)]
    bgd = bgt.to(DEV).requires_grad_() if bgt is not None else None
    rc, ra = _rasterize_to_pixels(ins[0], ins[1], ins[2], ins[3], W, H, ts, offs.to(DEV),
                                  fl.to(DEV), backgrounds=bgd, packed=packed,
                                  expected_depth_channel=D - 1)
    ((rc * v_rc.to(DEV)).sum() + (ra * v_ra.to(DEV)).sum()).backward()
    assert_close(rc.cpu(), outs["64"][0], RTOL, ATOL, "render_colors (ED)")
    for k, name in enumerate(("v_means2d", "v_conics", "v_colors", "v_opacities")):
        assert_grad_close(ins[k].grad, outs["64"][1][k].grad, outs["32"][1][k].grad,
                          RTOL, ATOL, name)
    if bg:
        assert_grad_close(bgd.grad, outs["64"][2].grad, outs["32"][2].grad, RTOL, ATOL,
                          "v_backgrounds")
        bgd = bgd.detach()
    with torch.no_grad():
        rc0, ra0 = rasterize_to_pixels(m2.to(DEV), con.to(DEV), col.to(DEV), op.to(DEV), W,
                                       H, ts, offs.to(DEV), fl.to(DEV), backgrounds=bgd,
                                       packed=packed)
        rc1, _ = _rasterize_to_pixels(m2.to(DEV), con.to(DEV), col.to(DEV), op.to(DEV), W,
                                      H, ts, offs.to(DEV), fl.to(DEV), backgrounds=bgd,
                                      packed=packed, expected_depth_channel=D - 1)
    want = ed(rc0, ra0).cpu().numpy()
    np.testing.assert_array_equal(rc.detach().cpu().numpy(), want)
    np.testing.assert_array_equal(rc1.cpu().numpy(), want)


@pytest.mark.parametrize("ed,packed", [(True, True), (False, True), (True, False)])
def test_separate_last_channel_matches_concatenated(ed, packed):
    """A last channel read from its own array (color_last: rasterization()'s
    depth channel kept apart from the colours) gives the render of the
    concatenated colours bit for bit, and their gradients, the last
    channel's split off, to float32 summation order (the flush's atomics add
    in any order)."""
    from gsplat_amd.cuda._wrapper import _rasterize_to_pixels
    data = projected_2d(seed=77, N=2000, C=2, D=4, packed=packed)
    W, H, ts, C = data["W"], data["H"], data["tile"], data["C"]
    offs, fl = data["offsets"].to(DEV), data["flatten_ids"].to(DEV)
    g = torch.Generator().manual_seed(9)
    bg = torch.rand(C, 4, generator=g).to(DEV)
    v_rc = torch.randn(C, H, W, 4, generator=g).to(DEV)
    v_ra = torch.randn(C, H, W, 1, generator=g).to(DEV)
    ch = 3 if ed else -1
    runs = []
    for split in (False, True):
        geo = [data[k].clone().to(DEV).requires_grad_()
               for k in ("means2d", "conics", "opacities")]
        col = data["colors"].to(DEV)
        if split:
            cols = [col[..., :3].contiguous().requires_grad_(),
                    col[..., 3].contiguous().requires_grad_()]
            rc, ra = _rasterize_to_pixels(geo[0], geo[1], cols[0], geo[2], W, H, ts, offs,
                                          fl, backgrounds=bg, packed=packed,
                                          expected_depth_channel=ch, color_last=cols[1])
        else:
            cols = [col.clone().requires_grad_()]
            rc, ra = _rasterize_to_pixels(geo[0], geo[1], cols[0], geo[2], W, H, ts, offs,
                                          fl, backgrounds=bg, packed=packed,
                                          expected_depth_channel=ch)
        ((rc * v_rc).sum() + (ra * v_ra).sum()).backward()
        v_col = (torch.cat([cols[0].grad, cols[1].grad[..., None]], dim=-1) if split
                 else cols[0].grad)
        runs.append((rc.detach(), ra.detach(), [t.grad for t in geo] + [v_col]))
    np.testing.assert_array_equal(runs[1][0].cpu().numpy(), runs[0][0].cpu().numpy())
    np.testing.assert_array_equal(runs[1][1].cpu().numpy(), runs[0][1].cpu().numpy())
    for name, a, b in zip(("v_means2d", "v_conics", "v_opacities", "v_colors"),
                          runs[0][2], runs[1][2]):
        assert bool(a.abs().sum() > 0), name
        assert_close(b.cpu(), a.cpu(), RTOL, ATOL, name)


def test_rasterize_backward_twice_through_retained_graph():
    """The forward zero-fills the backward's accumulators; the first backward
    adds into them and a second backward through the retained graph starts
    from fresh zeros: both give the same gradients."""
    from gsplat_amd.cuda._wrapper import rasterize_to_pixels
    data = projected_2d(seed=61, N=2000, C=2, D=3, packed=True)
    W, H, ts = data["W"], data["H"], data["tile"]
    ins = [data[k].clone().to(DEV).requires_grad_()
           for k in ("means2d", "conics", "colors", "opacities")]
    rc, ra = rasterize_to_pixels(ins[0], ins[1], ins[2], ins[3], W, H, ts,
                                 data["offsets"].to(DEV), data["flatten_ids"].to(DEV),
                                 packed=True)
    g = torch.Generator().manual_seed(4)
    loss = (rc * torch.randn(rc.shape, generator=g).to(DEV)).sum() + \
        (ra * torch.randn(ra.shape, generator=g).to(DEV)).sum()
    loss.backward(retain_graph=True)
    first = [t.grad.clone() for t in ins]
    for t in ins:
        t.grad = None
    loss.backward()
    for name, a, b in zip(("v_means2d", "v_conics", "v_colors", "v_opacities"),
                          first, (t.grad for t in ins)):
        assert bool(a.abs().sum() > 0), name
        assert_close(b.cpu(), a.cpu(), RTOL, ATOL, name)


def test_rasterize_unused_alpha_gradient():
    """A loss on the colours only: the alpha gradient reaches the backward as
    None (no zero tensor) and gives the same gradients as an explicit zero
    alpha gradient."""
    from gsplat_amd.cuda._wrapper import rasterize_to_pixels
    data = projected_2d(seed=60, N=2000, C=1, D=3)
    W, H, ts = data["W"], data["H"], data["tile"]
    grads = []
    for with_alpha in (False, True):
        ins = [data[k].clone().to(DEV).requires_grad_()
               for k in ("means2d", "conics", "colors", "opacities")]
        rc, ra = rasterize_to_pixels(ins[0], ins[1], ins[2], ins[3], W, H, ts,
                                     data["offsets"].to(DEV),
                                     data["flatten_ids"].to(DEV))
        g = torch.Generator().manual_seed(3)
        loss = (rc * torch.randn(rc.shape, generator=g).to(DEV)).sum()
        if with_alpha:
            loss = loss + (ra * 0.0).sum()
        loss.backward()
        grads.append([t.grad for t in ins])
    # tiles add their sums with float atomics in no fixed order: equal to
    # float32 rounding, not bit for bit
    for name, a, b in zip(("v_means2d", "v_conics", "v_colors", "v_opacities"),
                          *grads):
        assert_close(a.cpu(), b.cpu(), RTOL, ATOL, name)


def test_reference_schema_fwd_bwd_without_transmittance():
    """The reference's own autograd path (_wrapper.py:1709-1836) calls the
    schema ops: rasterize_to_pixels_3dgs_fwd, then rasterize_to_pixels_3dgs_bwd
    with render_alphas and last_ids only, so the backward takes the final
    transmittance as T' = 1 - render_alphas (RasterizeToPixels3DGSBwd.cu:130)
    instead of the forward's saved T.

    Every term of that backward is linear in the recovered transmittances
    (T_k = T' / prod_{j>=k} (1 - alpha_j), the colour buffer and T' itself), so
    its exact result is the exact gradient with each pixel's upstream
    gradients scaled by s = T' / T.  The oracle is therefore the float64
    restatement's autograd with v_render_colors and v_render_alphas scaled by
    s per pixel; the float32 restatement with the same scaling measures the
    fp32 floor."""
    data = projected_2d(seed=70, N=3000, C=2, D=3)
    W, H, ts, C, D = data["W"], data["H"], data["tile"], data["C"], 3
    m2, con, col, op = data["means2d"], data["conics"], data["colors"], data["opacities"]
    offs, fl = data["offsets"], data["flatten_ids"]
    g = torch.Generator().manual_seed(71)
    bg = torch.rand(C, D, generator=g)
    v_rc = torch.randn(C, H, W, D, generator=g)
    v_ra = torch.randn(C, H, W, 1, generator=g)

    ops = torch.ops.gsplat
    dev = [t.to(DEV) for t in (m2, con, col, op, bg, offs, fl)]
    rc, ra, last = ops.rasterize_to_pixels_3dgs_fwd(
        dev[0], dev[1], dev[2], dev[3], dev[4], None, W, H, ts, dev[5], dev[6])
    v_abs, v_m2, v_con, v_col, v_op = ops.rasterize_to_pixels_3dgs_bwd(
        dev[0], dev[1], dev[2], dev[3], dev[4], None, W, H, ts, dev[5], dev[6],
        ra, last, v_rc.to(DEV).contiguous(), v_ra.to(DEV).contiguous(), True)

    ins_ref = [t.double().requires_grad_() for t in (m2, con, col, op)]
    rc_r, ra_r, info = torch_ref.rasterize_to_pixels_ref(
        ins_ref[0], ins_ref[1], ins_ref[2], ins_ref[3], W, H, ts, offs, fl,
        backgrounds=bg.double())
    # forward outputs: decisions exact, colours within tolerance
    np.testing.assert_array_equal(last.cpu().numpy(), info["last_ids"])
    alpha32 = (np.float32(1.0) - info["transmittance"]).astype(np.float32)
    np.testing.assert_array_equal(ra.cpu().numpy()[..., 0], alpha32)
    assert_close(rc.cpu(), rc_r.detach(), RTOL, ATOL, "render_colors")

    t_saved = 1.0 - torch.from_numpy(alpha32.astype(np.float64))[..., None]
    s = (t_saved / (1.0 - ra_r.detach())).detach()
    ((rc_r * (v_rc.double() * s)).sum() + (ra_r * (v_ra.double() * s)).sum()).backward()
    ins32 = [t.float().clone().requires_grad_() for t in (m2, con, col, op)]
    rc32, ra32, _ = torch_ref.rasterize_to_pixels_ref(
        ins32[0], ins32[1], ins32[2], ins32[3], W, H, ts, offs, fl,
        backgrounds=bg.float(), dtype=torch.float32)
    s32 = s.float()
    ((rc32 * (v_rc * s32)).sum() + (ra32 * (v_ra * s32)).sum()).backward()
    for name, a, b, b32 in zip(("v_means2d", "v_conics", "v_colors", "v_opacities"),
                               (v_m2, v_con, v_col, v_op), ins_ref, ins32):
        print(assert_grad_close(a, b.grad, b32.grad, RTOL, ATOL, name))
    assert bool(torch.isfinite(v_abs).all())
    assert bool((v_abs + 1e-6 >= v_m2.abs()).all())
    # the scaling matters: pixels near the 1e-4 cutoff carry few bits of T'
    assert float((s - 1).abs().max()) > 1e-5


def _direct_grads(data, D, bg, mk, v_rc, v_ra, replay):
    """Gradients through the C-ABI ops directly: the forward with its saved
    transmittance, then either the per-batch replay (rasterize_bwd_replay,
    what rasterization() runs) or the whole-tile replay from T."""
    from gsplat_amd.cuda import _ops
    W, H, ts = data["W"], data["H"], data["tile"]
    ins = [data[k].to(DEV) for k in ("means2d", "conics", "colors", "opacities")]
    bgd = bg.to(DEV) if bg is not None else None
    mkd = mk.to(DEV) if mk is not None else None
    offs, fl = data["offsets"].to(DEV), data["flatten_ids"].to(DEV)
    if replay:
        rc, ra, last, T, state = _ops.rasterize_fwd_replay(
            *ins, bgd, mkd, W, H, ts, offs, fl)
        grads = _ops.rasterize_bwd_replay(
            *ins, bgd, mkd, W, H, ts, offs, fl, T, last, state, v_rc.to(DEV),
            v_ra.to(DEV), False)
        n_units = int(state.records[:4].cpu().view(torch.int32)[0])
    else:
        rc, ra, last, T = _ops.rasterize_fwd_with_transmittance(
            *ins, bgd, mkd, W, H, ts, offs, fl)
        grads = _ops.rasterize_to_pixels_3dgs_bwd(
            *ins, bgd, mkd, W, H, ts, offs, fl, ra, last, v_rc.to(DEV),
            v_ra.to(DEV), False, render_transmittance=T)
        n_units = None
    torch.cuda.synchronize()
    return rc, ra, grads[1:], n_units


@pytest.mark.parametrize("D,tile", [(3, 16), (3, 8), (4, 16), (32, 16)])
def test_replay_units_match_oracle_on_deep_tiles(D, tile):
    """Deep tiles (many faint, large Gaussians: several forward batches per
    tile and pixels that stay unsaturated) through the per-batch units that
    start from the forward's records, held to the oracle's gradients; the
    units must really split tiles (more units than tiles).

    The whole-tile replay from the final T runs too, for the renders only: on
    such tiles it recovers each T by dividing the final float32 T back over
    hundreds of Gaussians, which cannot undo the forward's float32 roundings
    of the steps behind, and its conic gradients drift past the float32
    restatement's (3.2x its worst element at tile 8).  The units restart
    from the forward's own T at every batch boundary."""
    data = projected_2d(seed=70 + D + tile, N=3000, C=1, W=96, H=64, tile=tile, D=D,
                        opac_range=(0.02, 0.2), scale_range=(0.05, 0.3), spread=0.8)
    W, H, ts, C = data["W"], data["H"], data["tile"], data["C"]
    g = torch.Generator().manual_seed(5)
    bg = torch.rand(C, D, generator=g)
    mk = torch.rand(data["offsets"].shape, generator=g) > 0.15
    v_rc = torch.randn(C, H, W, D, generator=g)
    v_ra = torch.randn(C, H, W, 1, generator=g)
    m2, con, col, op = (data[k] for k in ("means2d", "conics", "colors", "opacities"))
    ins_ref = [t.double().requires_grad_() for t in (m2, con, col, op)]
    rc_r, ra_r, info = torch_ref.rasterize_to_pixels_ref(
        *ins_ref, W, H, ts, data["offsets"], data["flatten_ids"],
        backgrounds=bg.double(), masks=mk)
    ((rc_r * v_rc.double()).sum() + (ra_r * v_ra.double()).sum()).backward()
    ins32 = [t.float().clone().requires_grad_() for t in (m2, con, col, op)]
    rc32, ra32, _ = torch_ref.rasterize_to_pixels_ref(
        *ins32, W, H, ts, data["offsets"], data["flatten_ids"],
        backgrounds=bg.float(), masks=mk, dtype=torch.float32)
    ((rc32 * v_rc).sum() + (ra32 * v_ra).sum()).backward()
    alpha32 = (np.float32(1.0) - info["transmittance"]).astype(np.float32)
    n_tiles = int(mk.sum())
    per_tile = np.diff(np.append(data["offsets"].numpy().ravel(),
                                 data["flatten_ids"].numel()))
    assert per_tile.max() > 3 * tile * tile, "scene too shallow for several batches"
    for replay in (True, False):
        rc, ra, grads, n_units = _direct_grads(data, D, bg, mk, v_rc, v_ra, replay)
        np.testing.assert_array_equal(ra.cpu().numpy()[..., 0], alpha32)
        assert_close(rc.cpu(), rc_r.detach(), RTOL, ATOL, "render_colors")
        if not replay:
            continue
        assert n_units > n_tiles, (n_units, n_tiles)
        for name, a, b, b32 in zip(("v_means2d", "v_conics", "v_colors", "v_opacities"),
                                   grads, ins_ref, ins32):
            assert_grad_close(a, b.grad, b32.grad, RTOL, ATOL, name)


def _thin_ellipses_everywhere(seed, N, W, H, tile, D):
    """N thin, rotated 2D Gaussians (axis ratios up to 1:60, support from a
    fraction of a pixel to ~40 px) over and around a W x H image, each listed
    in every tile in one depth order, so every (Gaussian, tile, strip)
    combination reaches the rasterizers' strip masks; a quarter of the
    centres sit on pixel centres or strip boundaries."""
    g = torch.Generator().manual_seed(seed)
    th = torch.rand(N, generator=g, dtype=torch.float64) * math.pi
    s_major = 0.3 + 12.0 * torch.rand(N, generator=g, dtype=torch.float64)
    s_minor = s_major / (1.0 + 59.0 * torch.rand(N, generator=g, dtype=torch.float64))
    cos, sin = torch.cos(th), torch.sin(th)
    # covariance R diag(s^2) R^T, conic = its inverse
    a11 = cos ** 2 * s_major ** 2 + sin ** 2 * s_minor ** 2
    a22 = sin ** 2 * s_major ** 2 + cos ** 2 * s_minor ** 2
    a12 = cos * sin * (s_major ** 2 - s_minor ** 2)
    det = a11 * a22 - a12 ** 2
    conics = torch.stack([a22 / det, -a12 / det, a11 / det], -1).float()
    means = torch.rand(N, 2, generator=g, dtype=torch.float64)
    means = means * torch.tensor([W + 24.0, H + 24.0], dtype=torch.float64) - 12.0
    k = N // 4
    snap = torch.randint(0, 4, (k, 2), generator=g).double()
    means[:k] = torch.floor(means[:k] / 4.0) * 4.0 + snap * 0.5  # centres and edges
    opac = (0.01 + 0.99 * torch.rand(N, generator=g)).float()
    colors = torch.rand(1, N, D, generator=g)
    order = torch.randperm(N, generator=g).to(torch.int32)
    tw, th_ = math.ceil(W / tile), math.ceil(H / tile)
    flatten = order.repeat(tw * th_)
    offsets = (torch.arange(tw * th_, dtype=torch.int32) * N).reshape(1, th_, tw)
    return {
        "means2d": means.float()[None].contiguous(), "conics": conics[None].contiguous(),
        "opacities": opac[None].contiguous(), "colors": colors.contiguous(),
        "offsets": offsets, "flatten_ids": flatten, "W": W, "H": H, "tile": tile, "C": 1,
    }


@pytest.mark.parametrize("tile", [16, 8])
def test_strip_culling_keeps_every_pixel_of_thin_rotated_ellipses(tile):
    """Each rasterizer wave skips the Gaussians whose ellipse misses its pixel
    strip (the minimum of the quadratic form over the strip against the
    alpha threshold).  A skip that dropped one composited pixel would change
    that pixel's alpha and last contributor, which are compared bit for bit
    here over thin ellipses at every angle in every tile; the gradients are
    held to the oracle as everywhere else."""
    data = _thin_ellipses_everywhere(seed=90 + tile, N=400, W=64, H=48, tile=tile, D=3)
    ins = _run(data, False, 3, backgrounds=False, masks=False)
    assert all(bool(torch.isfinite(t.grad).all()) for t in ins)
    from gsplat_amd.cuda import _ops
    _, _, info = torch_ref.rasterize_to_pixels_ref(
        *(data[k].double() for k in ("means2d", "conics", "colors", "opacities")),
        data["W"], data["H"], tile, data["offsets"], data["flatten_ids"])
    _, _, last = _ops.rasterize_to_pixels_3dgs_fwd(
        *(data[k].to(DEV) for k in ("means2d", "conics", "colors", "opacities")),
        None, None, data["W"], data["H"], tile, data["offsets"].to(DEV),
        data["flatten_ids"].to(DEV))
    np.testing.assert_array_equal(last.cpu().numpy(), info["last_ids"])
