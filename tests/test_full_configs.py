"""BASELINE configurations 1 to 4 at their full sizes on the GPU, through
``rasterization()`` (gsplat/rendering.py:256-1273), against the host oracle.

Every full-size run is checked on all of its intersections: ``isect_ids``,
``flatten_ids`` and the tile offsets bit-exact against the oracle's
intersection of the oracle's projection (C restatement).  Pixels are checked on
a strided sample of tiles, where the oracle composites exactly the Gaussians
the kernels do: ``render_alphas`` bit-exact (1 - T with T the float32 running
product), colours within rtol 1e-4 / atol 1e-5 of the float64 restatement.
Gradients (configs 1, 2 and 4) come from an upstream gradient that is nonzero on
the sampled tiles only, so the oracle's autograd over those tiles gives the
whole gradient; they are held to rtol 1e-4 / atol 1e-5 at the float32 floor
(tests/_util.py:assert_grad_close) over every Gaussian the sample touches.
Config 4 also checks the densification statistics on the step's own absgrad
and the fused Adam update of all 118M parameter elements bit for bit."""

import math

import numpy as np
import pytest
import torch

from gsplat_amd._helper import make_scene
from oracle import exact, torch_ref
from tests._util import DEV, assert_close, assert_grad_close

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-5
TILE = 16


def _tile_sample(C, th, tw, stride, start=5):
    return np.arange(start, C * th * tw, stride)


def _pixel_mask(C, H, W, th, tw, sample):
    m = np.zeros((C, th * TILE, tw * TILE), bool)
    for slot in sample:
        img, t = divmod(int(slot), th * tw)
        ty, tx = divmod(t, tw)
        m[img, ty * TILE:(ty + 1) * TILE, tx * TILE:(tx + 1) * TILE] = True
    return torch.from_numpy(np.ascontiguousarray(m[:, :H, :W]))


def _oracle(params, transform, scene, sample, dtype, v_rc, v_ra, backward):
    """Oracle render on the tile sample (rows restricted to the sample's);
    returns (rc, ra, meta, leaf gradients or None)."""
    leaves = {k: v.detach().clone().to(dtype).requires_grad_(backward)
              for k, v in params.items()}
    means, quats, scales, opac, colors = transform(leaves)
    rc, ra, meta = torch_ref.rasterization_ref(
        means, quats, scales, opac, colors, scene.viewmats, scene.Ks, scene.width,
        scene.height, sh_degree=scene.sh_degree, dtype=dtype, tile_subset=sample,
        restrict_rows=True, **scene.kwargs)
    grads = None
    if backward:
        ((rc * v_rc.to(dtype)).sum() + (ra * v_ra.to(dtype)).sum()).backward()
        grads = {k: v.grad for k, v in leaves.items()}
    return rc.detach(), ra.detach(), meta, grads


def _check_forward(meta, rc, ra, meta_r, rc_r, ra_r, pix):
    np.testing.assert_array_equal(meta["isect_ids"].cpu().numpy(), meta_r["isect_ids"])
    np.testing.assert_array_equal(meta["flatten_ids"].cpu().numpy(), meta_r["flatten_ids"])
    np.testing.assert_array_equal(meta["isect_offsets"].cpu().numpy().reshape(-1),
                                  meta_r["offsets"].reshape(-1))
    alpha32 = (np.float32(1.0) - meta_r["transmittance"]).astype(np.float32)
    got_a = ra.detach().cpu().numpy()[..., 0]
    p = pix.numpy()
    np.testing.assert_array_equal(got_a[p], alpha32[p])
    assert_close(rc.detach().cpu()[pix], rc_r[pix], RTOL, ATOL, "render_colors")
    assert_close(ra.detach().cpu()[pix], ra_r[pix], RTOL, ATOL, "render_alphas")
    assert float(ra_r[pix].max()) > 0.5  # the sample is not empty sky


def _check_grads(got, ref64, ref32):
    for k in got:
        r = ref64[k].reshape(ref64[k].shape[0], -1)
        touched = (r != 0).any(dim=1)
        assert int(touched.sum()) > 100, k
        print(assert_grad_close(got[k][touched], ref64[k][touched], ref32[k][touched],
                                RTOL, ATOL, f"d{k}"))


def _plain(leaves):
    return (leaves["means"], leaves["quats"], leaves["scales"], leaves["opacities"],
            leaves["colors"])


def test_cfg1_full_size_fwd_bwd_queued_stage():
    """1M Gaussians, SH3, 1280x720, packed, fwd+bwd.  Two calls: the second
    queues the sorted emission with the count read on the device, sized from
    the first call's count (the path the timed benchmark steps take)."""
    import gsplat_amd as gs
    from gsplat_amd.cuda import _ops
    scene = make_scene(1)
    C, H, W = 1, scene.height, scene.width
    th, tw = math.ceil(H / TILE), math.ceil(W / TILE)
    sample = _tile_sample(C, th, tw, 61)
    pix = _pixel_mask(C, H, W, th, tw, sample)
    g = torch.Generator().manual_seed(1)
    v_rc = torch.randn(C, H, W, 3, generator=g) * pix[..., None]
    v_ra = torch.randn(C, H, W, 1, generator=g) * pix[..., None]
    params = {k: getattr(scene, k) for k in ("means", "quats", "scales", "opacities",
                                             "colors")}
    rc_r, ra_r, meta_r, g64 = _oracle(params, _plain, scene, sample, torch.float64,
                                      v_rc, v_ra, True)
    _, _, _, g32 = _oracle(params, _plain, scene, sample, torch.float32, v_rc, v_ra, True)
    assert meta_r["n_isects"] > 4_000_000

    for call in range(2):
        gl = {k: v.to(DEV).requires_grad_() for k, v in params.items()}
        if call == 1:
            cap = _ops.isect_capacity(torch.device(DEV))
            assert cap is not None and cap >= meta_r["n_isects"]
        rc, ra, meta = gs.rasterization(gl["means"], gl["quats"], gl["scales"],
                                        gl["opacities"], gl["colors"],
                                        scene.viewmats.to(DEV), scene.Ks.to(DEV), W, H,
                                        sh_degree=3)
        ((rc * v_rc.to(DEV)).sum() + (ra * v_ra.to(DEV)).sum()).backward()
        print(f"[cfg1] call {call}: {meta['isect_ids'].numel()} intersections", flush=True)
        _check_forward(meta, rc, ra, meta_r, rc_r, ra_r, pix)
    _check_grads({k: v.grad.cpu() for k, v in gl.items()}, g64, g32)


def test_cfg2_full_size_rgb_ed_fwd_bwd():
    """500k Gaussians, SH1, 8 cameras on a ring (960x540 each), packed,
    render mode RGB+ED (the expected depth divided inside the rasterizer),
    fwd+bwd: all 12M intersections over the 8 images bit-exact, pixels and
    gradients on a tile sample spread over every camera."""
    import gsplat_amd as gs
    scene = make_scene(2)
    C, H, W = scene.viewmats.shape[0], scene.height, scene.width
    th, tw = math.ceil(H / TILE), math.ceil(W / TILE)
    sample = _tile_sample(C, th, tw, 211)
    assert len(np.unique(sample // (th * tw))) == C
    pix = _pixel_mask(C, H, W, th, tw, sample)
    g = torch.Generator().manual_seed(2)
    v_rc = torch.randn(C, H, W, 4, generator=g) * pix[..., None]
    v_ra = torch.randn(C, H, W, 1, generator=g) * pix[..., None]
    params = {k: getattr(scene, k) for k in ("means", "quats", "scales", "opacities",
                                             "colors")}
    rc_r, ra_r, meta_r, g64 = _oracle(params, _plain, scene, sample, torch.float64,
                                      v_rc, v_ra, True)
    _, _, _, g32 = _oracle(params, _plain, scene, sample, torch.float32, v_rc, v_ra, True)
    assert meta_r["n_isects"] > 10_000_000

    gl = {k: v.to(DEV).requires_grad_() for k, v in params.items()}
    rc, ra, meta = gs.rasterization(gl["means"], gl["quats"], gl["scales"],
                                    gl["opacities"], gl["colors"],
                                    scene.viewmats.to(DEV), scene.Ks.to(DEV), W, H,
                                    sh_degree=scene.sh_degree, **scene.kwargs)
    assert rc.shape == (C, H, W, 4)
    ((rc * v_rc.to(DEV)).sum() + (ra * v_ra.to(DEV)).sum()).backward()
    print(f"[cfg2] {meta['isect_ids'].numel()} intersections", flush=True)
    _check_forward(meta, rc, ra, meta_r, rc_r, ra_r, pix)
    _check_grads({k: v.grad.cpu() for k, v in gl.items()}, g64, g32)


def test_cfg3_full_size_forward():
    """6M Gaussians in a 40x10x40 box around the camera, heavy-tailed scales,
    SH3, 1920x1080 (13-bit tile keys), forward only."""
    import gsplat_amd as gs
    scene = make_scene(3)
    C, H, W = 1, scene.height, scene.width
    th, tw = math.ceil(H / TILE), math.ceil(W / TILE)
    assert (th * tw).bit_length() == 13
    sample = _tile_sample(C, th, tw, 97)
    pix = _pixel_mask(C, H, W, th, tw, sample)
    params = {k: getattr(scene, k) for k in ("means", "quats", "scales", "opacities",
                                             "colors")}
    rc_r, ra_r, meta_r, _ = _oracle(params, _plain, scene, sample, torch.float64,
                                    None, None, False)
    with torch.no_grad():
        d = {k: v.to(DEV) for k, v in params.items()}
        rc, ra, meta = gs.rasterization(d["means"], d["quats"], d["scales"],
                                        d["opacities"], d["colors"],
                                        scene.viewmats.to(DEV), scene.Ks.to(DEV), W, H,
                                        sh_degree=3)
    print(f"[cfg3] {meta['isect_ids'].numel()} intersections, "
          f"{meta['means2d'].shape[0]} visible rows", flush=True)
    _check_forward(meta, rc, ra, meta_r, rc_r, ra_r, pix)


def _cfg4_transform(leaves, snap=None):
    """Raw parameters -> rasterization() inputs.  ``snap`` holds the float32
    scales and opacities the GPU computed (exp and sigmoid may round
    differently on the host): the host values are replaced by those exact
    values while the gradient still flows through exp and sigmoid, so the
    oracle decides on the same float32 inputs the kernels see."""
    colors = torch.cat([leaves["sh0"], leaves["shN"]], dim=1)
    scales = leaves["log_scales"].exp()
    opac = torch.sigmoid(leaves["opacity_logits"])
    if snap is not None:
        scales = scales + (snap["scales"].to(scales.dtype) - scales).detach()
        opac = opac + (snap["opacities"].to(opac.dtype) - opac).detach()
    return leaves["means"], leaves["quats"], scales, opac, colors


def test_cfg4_full_size_optimizer_step():
    """2M Gaussians, SH3, 1600x1040: fwd+bwd on the raw parameters with
    absgrad, the densification statistics, and the fused Adam step over the
    six tensors (118M elements, the config's learning rates)."""
    import gsplat_amd as gs
    from gsplat_amd.cuda import _ops
    from gsplat_amd.strategy.stats import accumulate_grad2d_stats, fuse_grad2d_stats
    scene = make_scene(4)
    C, H, W = 1, scene.height, scene.width
    N = scene.means.shape[0]
    th, tw = math.ceil(H / TILE), math.ceil(W / TILE)
    sample = _tile_sample(C, th, tw, 101)
    pix = _pixel_mask(C, H, W, th, tw, sample)
    g = torch.Generator().manual_seed(4)
    v_rc = torch.randn(C, H, W, 3, generator=g) * pix[..., None]
    v_ra = torch.randn(C, H, W, 1, generator=g) * pix[..., None]
    raw = {"means": scene.means, "log_scales": scene.log_scales, "quats": scene.quats,
           "opacity_logits": scene.opacity_logits, "sh0": scene.colors[:, :1].contiguous(),
           "shN": scene.colors[:, 1:].contiguous()}
    params = {k: v.to(DEV).requires_grad_() for k, v in raw.items()}
    with torch.no_grad():
        snap = {"scales": params["log_scales"].exp().cpu(),
                "opacities": torch.sigmoid(params["opacity_logits"]).cpu()}
    transform = lambda leaves: _cfg4_transform(leaves, snap)
    rc_r, ra_r, meta_r, g64 = _oracle(raw, transform, scene, sample, torch.float64,
                                      v_rc, v_ra, True)
    _, _, _, g32 = _oracle(raw, transform, scene, sample, torch.float32, v_rc, v_ra, True)

    means, quats, scales, opac, colors = _cfg4_transform(params)
    rc, ra, meta = gs.rasterization(means, quats, scales, opac, colors,
                                    scene.viewmats.to(DEV), scene.Ks.to(DEV), W, H,
                                    sh_degree=3, absgrad=True)
    # densification statistics accumulated by the projection backward, onto a
    # running state, as bench.py --config 4 takes them
    gs_ = torch.Generator().manual_seed(6)
    prev_g = torch.rand(N, generator=gs_)
    prev_c = torch.randint(0, 5, (N,), generator=gs_).float()
    grad2d, count, fused = fuse_grad2d_stats(meta, prev_g.to(DEV), prev_c.to(DEV), N,
                                             absgrad=True)
    assert fused
    ((rc * v_rc.to(DEV)).sum() + (ra * v_ra.to(DEV)).sum()).backward()
    print(f"[cfg4] {meta['isect_ids'].numel()} intersections", flush=True)
    _check_forward(meta, rc, ra, meta_r, rc_r, ra_r, pix)
    _check_grads({k: v.grad.cpu() for k, v in params.items()}, g64, g32)

    # the statistics of the step's own absgrad (strategy/default.py:235-268)
    absgrad = meta["means2d"].absgrad.detach().cpu()
    assert float(absgrad.abs().sum()) > 0
    r_g, r_c = torch_ref.grad2d_stats_ref(absgrad, meta["gaussian_ids"].cpu(), None, N, W,
                                         H, C, prev_g, prev_c)
    assert torch.equal(count.cpu().double(), r_c)
    assert_close(grad2d.cpu(), r_g, 1e-5, 1e-9, "grad2d (fused)")
    # and the separate pass over the same rows from zero
    sep_g, sep_c = accumulate_grad2d_stats(meta, None, None, N, packed=True, absgrad=True)
    r_g0, r_c0 = torch_ref.grad2d_stats_ref(absgrad, meta["gaussian_ids"].cpu(), None, N,
                                           W, H, C)
    assert torch.equal(sep_c.cpu().double(), r_c0)
    assert_close(sep_g.cpu(), r_g0, 1e-5, 1e-9, "grad2d (separate)")

    # fused Adam over all six tensors from a nonzero state, bit for bit
    lrs = {"means": 1.6e-4, "log_scales": 5e-3, "quats": 1e-3, "opacity_logits": 5e-2,
           "sh0": 2.5e-3, "shN": 1.25e-4}
    gm = torch.Generator().manual_seed(5)
    state = {}
    for k, p in params.items():
        m = torch.randn(p.shape, generator=gm) * 1e-3
        v = torch.rand(p.shape, generator=gm) * 1e-6
        state[k] = (m, v)
    host = {k: (p.detach().cpu().numpy(), p.grad.cpu().numpy()) for k, p in params.items()}
    dev_state = {k: (m.to(DEV), v.to(DEV)) for k, (m, v) in state.items()}
    with torch.no_grad():
        _ops.adam_multi([(params[k], params[k].grad, dev_state[k][0], dev_state[k][1],
                          None, lrs[k]) for k in params], 0.9, 0.999, 1e-15)
    torch.cuda.synchronize()
    n_elem = 0
    for k in params:
        p_np, g_np = host[k]
        pn, mn, vn = exact.adam(p_np, g_np, state[k][0].numpy(), state[k][1].numpy(), None,
                                lrs[k], 0.9, 0.999, 1e-15)
        np.testing.assert_array_equal(params[k].detach().cpu().numpy().view(np.uint32),
                                      pn.view(np.uint32))
        np.testing.assert_array_equal(dev_state[k][0].cpu().numpy().view(np.uint32),
                                      mn.view(np.uint32))
        np.testing.assert_array_equal(dev_state[k][1].cpu().numpy().view(np.uint32),
                                      vn.view(np.uint32))
        n_elem += p_np.size
    assert n_elem == N * (3 + 3 + 4 + 1 + 3 + 45)
