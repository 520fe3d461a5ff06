"""Pins the host oracle itself (CPU only): closed forms, brute force,
invariants and cross-checks between its two independent restatements.

A wrong sign, index or dropped term in the oracle fails one of these."""

import math

import numpy as np
import pytest
import torch

from oracle import exact, torch_ref


# --------------------------------------------------------------------------
# log
# --------------------------------------------------------------------------
def test_portable_log_numpy_equals_c_and_is_accurate():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.uniform(0, 300, 50_000), 10 ** rng.uniform(-44, 38, 50_000),
        [1.0, 255.0, 1e-45, 3.4e38],
    ]).astype(np.float32)
    a = exact.portable_logf(x)
    b = exact.portable_logf_c(x)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    ref = np.log(x.astype(np.float64))
    ulp = np.abs(a - ref) / np.spacing(np.abs(ref).astype(np.float32))
    assert ulp.max() < 2.0
    special = exact.portable_logf(np.array([0.0, -1.0, np.inf, np.nan], np.float32))
    assert np.isnan(special[0]) and np.isnan(special[1]) and special[2] == np.inf
    assert np.isnan(special[3])


# --------------------------------------------------------------------------
# exp (the alpha of every composited pixel/Gaussian pair)
# --------------------------------------------------------------------------
def test_portable_exp_is_accurate():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        np.linspace(-87.0, 88.0, 400_001), rng.uniform(-6.0, 0.0, 200_000),
        -np.arange(0, 126) * np.log(2.0),
    ]).astype(np.float32)
    y = exact.portable_expf(x)
    ref = np.exp(x.astype(np.float64))
    ulp = np.abs(y - ref) / np.spacing(ref.astype(np.float32)).astype(np.float64)
    # below 1 ulp everywhere (a dropped Taylor term or a one-part ln2 fails this)
    assert ulp.max() < 1.0, ulp.max()
    assert exact.portable_expf(np.float32(0.0)) == np.float32(1.0)
    special = exact.portable_expf(np.array([-100.0, 100.0, np.nan], np.float32))
    assert special[0] == 0.0 and special[1] == np.inf and np.isnan(special[2])


# --------------------------------------------------------------------------
# Projection
# --------------------------------------------------------------------------
def _axis_gaussian(z=4.0, s=0.05, f=300.0, W=200, H=100, opacity=None):
    means = np.array([[0.0, 0.0, z]], np.float32)
    quats = np.array([[1.0, 0.0, 0.0, 0.0]], np.float32)
    scales = np.full((1, 3), s, np.float32)
    vm = np.eye(4, dtype=np.float32)[None]
    K = np.array([[[f, 0, W / 2], [0, f, H / 2], [0, 0, 1]]], np.float32)
    op = None if opacity is None else np.array([opacity], np.float32)
    return means, quats, scales, op, vm, K, W, H


def test_projection_closed_form_isotropic_on_axis():
    z, s, f, W, H = 4.0, 0.05, 300.0, 200, 100
    means, quats, scales, op, vm, K, W, H = _axis_gaussian(z, s, f, W, H)
    out = exact.projection_fwd(means, None, quats, scales, op, vm, K, W, H,
                               calc_compensations=True)
    var = (f * s / z) ** 2
    assert out["valid"][0, 0]
    np.testing.assert_allclose(out["means2d"][0, 0], [W / 2, H / 2], rtol=1e-6)
    np.testing.assert_allclose(out["depths"][0, 0], z, rtol=1e-6)
    np.testing.assert_allclose(out["conics"][0, 0], [1 / (var + 0.3), 0.0, 1 / (var + 0.3)],
                               rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(out["compensations"][0, 0], var / (var + 0.3), rtol=1e-5)
    r = math.ceil(3.33 * math.sqrt(var + 0.3))
    assert tuple(out["radii"][0, 0]) == (r, r)
    # the float restatement agrees
    t = torch_ref.projection_ref(torch.tensor(means, dtype=torch.float64), None,
                                 torch.tensor(quats, dtype=torch.float64),
                                 torch.tensor(scales, dtype=torch.float64),
                                 torch.tensor(vm, dtype=torch.float64),
                                 torch.tensor(K, dtype=torch.float64), W, H,
                                 calc_compensations=True)
    np.testing.assert_allclose(t["conics"][0, 0].numpy(), out["conics"][0, 0], rtol=1e-5, atol=1e-8)
    np.testing.assert_allclose(t["compensations"][0, 0].numpy(), var / (var + 0.3), rtol=1e-7)


def test_projection_opacity_aware_radius_closed_form():
    z, s, f, W, H = 4.0, 0.05, 300.0, 200, 100
    for o in (0.02, 0.5, 1.0):
        means, quats, scales, op, vm, K, W, H = _axis_gaussian(z, s, f, W, H, o)
        out = exact.projection_fwd(means, None, quats, scales, op, vm, K, W, H)
        var = (f * s / z) ** 2 + 0.3
        ext = min(3.33, math.sqrt(2 * math.log(o * 255.0)))
        r = math.ceil(ext * math.sqrt(var))
        assert tuple(out["radii"][0, 0]) == (r, r), (o, out["radii"][0, 0], r)
    # below 1/255 the row is culled
    means, quats, scales, op, vm, K, W, H = _axis_gaussian(opacity=1.0 / 256)
    assert not exact.projection_fwd(means, None, quats, scales, op, vm, K, W, H)["valid"].any()


@pytest.mark.parametrize("case", ["near", "far", "offimage", "clip"])
def test_projection_culling_cases(case):
    means, quats, scales, op, vm, K, W, H = _axis_gaussian()
    kw = {}
    if case == "near":
        means[0, 2] = 0.005
    elif case == "far":
        kw["far_plane"] = 3.0
    elif case == "offimage":
        means[0, 0] = 10.0
    elif case == "clip":
        kw["radius_clip"] = 100.0
    out = exact.projection_fwd(means, None, quats, scales, op, vm, K, W, H, **kw)
    assert not out["valid"].any()
    assert (out["radii"] == 0).all() and (out["conics"] == 0).all()


def _random_scene(seed=0, N=3000, C=2):
    g = torch.Generator().manual_seed(seed)
    means = torch.randn(N, 3, generator=g) * 1.5
    quats = torch.randn(N, 4, generator=g)
    scales = torch.rand(N, 3, generator=g) * 0.1 + 0.005
    opac = torch.rand(N, generator=g)
    vms = []
    for k in range(C):
        th = 0.4 * k
        from gsplat_amd._helper import look_at_viewmat
        vms.append(look_at_viewmat((5 * math.sin(th), -0.5, -5 * math.cos(th))))
    vm = torch.stack(vms)
    K = torch.tensor([[300.0, 0, 160], [0, 300.0, 120], [0, 0, 1]]).expand(C, 3, 3).contiguous()
    return means, quats, scales, opac, vm, K, 320, 240


def test_projection_exact_oracle_matches_float_restatement():
    means, quats, scales, opac, vm, K, W, H = _random_scene()
    ex = exact.projection_fwd(means.numpy(), None, quats.numpy(), scales.numpy(),
                              opac.numpy(), vm.numpy(), K.numpy(), W, H,
                              calc_compensations=True)
    t = torch_ref.projection_ref(means.double(), None, quats.double(), scales.double(),
                                 vm.double(), K.double(), W, H, calc_compensations=True,
                                 opacities=opac.double())
    v = ex["valid"]
    tv = t["valid"].numpy()
    # visibility agrees except for rows whose float radius sits on a ceil or
    # image-border boundary
    assert (v != tv).mean() < 2e-3
    both = v & tv
    np.testing.assert_allclose(ex["means2d"][both], t["means2d"].numpy()[both], rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(ex["depths"][both], t["depths"].numpy()[both], rtol=1e-6)
    np.testing.assert_allclose(ex["conics"][both], t["conics"].numpy()[both], rtol=2e-4, atol=1e-6)
    np.testing.assert_allclose(ex["compensations"][both], t["compensations"].numpy()[both],
                               rtol=2e-4, atol=1e-6)
    dr = np.abs(ex["radii"][both] - t["radius_f"].numpy()[both])
    assert dr.max() <= 1 and (dr > 0).mean() < 2e-3


def test_projection_float_restatement_grad_matches_finite_differences():
    means, quats, scales, opac, vm, K, W, H = _random_scene(N=20, C=1)
    params = [means.double().requires_grad_(), quats.double().requires_grad_(),
              scales.double().requires_grad_()]
    wts = torch.randn(20, 6, dtype=torch.float64)

    def f(m, q, s):
        t = torch_ref.projection_ref(m, None, q, s, vm.double(), K.double(), W, H)
        y = torch.cat([t["means2d"][0], t["conics"][0], t["depths"][0, :, None]], dim=-1)
        return (y * wts).sum()

    assert torch.autograd.gradcheck(f, params, eps=1e-6, atol=1e-5, rtol=1e-4)


# --------------------------------------------------------------------------
# Tile intersection
# --------------------------------------------------------------------------
def test_isect_box_matches_reference_loop():
    """Box path against the loop form of the reference's own oracle
    (tests/test_basic.py:698-736 inputs: C=3, N=1000, 40x60 image)."""
    rng = np.random.default_rng(42)
    C, N, W, H, ts = 3, 1000, 40, 60, 16
    means2d = (rng.standard_normal((C, N, 2)) * W).astype(np.float32)
    radii = rng.integers(0, W, (C, N, 2)).astype(np.int32)
    depths = rng.random((C, N)).astype(np.float32)
    tw, th = math.ceil(W / ts), math.ceil(H / ts)
    a = exact.isect_tiles(means2d, radii, depths, ts, tw, th)
    b = exact.isect_tiles_box_python(means2d, radii, depths, ts, tw, th)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    offs = exact.isect_offset_encode(a[1], C, tw, th)
    # brute force: offsets[i, t] = number of keys with (image, tile) < (i, t)
    hi = a[1] >> 32
    tb = (tw * th).bit_length()
    for i in range(C):
        for t in range(tw * th):
            assert offs.reshape(C, -1)[i, t] == int(np.sum(hi < ((i << tb) | t)))


def _ellipse_rows(seed=1, n=400, W=200, H=150):
    rng = np.random.default_rng(seed)
    mean = np.stack([rng.uniform(-20, W + 20, n), rng.uniform(-20, H + 20, n)], -1).astype(np.float32)
    # random SPD 2D covariances -> conics
    ang = rng.uniform(0, np.pi, n)
    s1 = rng.uniform(1, 30, n)
    s2 = rng.uniform(1, 30, n)
    c, s = np.cos(ang), np.sin(ang)
    cov = np.empty((n, 2, 2))
    cov[:, 0, 0] = c * c * s1 ** 2 + s * s * s2 ** 2
    cov[:, 1, 1] = s * s * s1 ** 2 + c * c * s2 ** 2
    cov[:, 0, 1] = cov[:, 1, 0] = c * s * (s1 ** 2 - s2 ** 2)
    inv = np.linalg.inv(cov)
    conics = np.stack([inv[:, 0, 0], inv[:, 0, 1], inv[:, 1, 1]], -1).astype(np.float32)
    opac = rng.uniform(0.01, 1.0, n).astype(np.float32)
    ext = np.minimum(3.33, np.sqrt(2 * np.log(opac * 255.0)))
    radii = np.ceil(ext[:, None] * np.sqrt(np.stack([cov[:, 0, 0], cov[:, 1, 1]], -1))).astype(np.int32)
    depths = rng.uniform(1, 10, n).astype(np.float32)
    return mean, radii, depths, conics, opac


def test_accutile_subset_of_box_and_covers_level_set():
    W, H, ts = 200, 150, 16
    tw, th = math.ceil(W / ts), math.ceil(H / ts)
    mean, radii, depths, conics, opac = _ellipse_rows(W=W, H=H)
    n = mean.shape[0]
    acc = exact.isect_tiles(mean[None], radii[None], depths[None], ts, tw, th, sort=False,
                            conics=conics[None], opacities=opac[None])
    box = exact.isect_tiles(mean[None], radii[None], depths[None], ts, tw, th, sort=False)
    assert acc[1].shape[0] < box[1].shape[0]
    tb = (tw * th).bit_length()
    acc_sets = [set() for _ in range(n)]
    for k, f in zip(acc[1], acc[2]):
        acc_sets[f].add(int((k >> 32) & ((1 << tb) - 1)))
    box_sets = [set() for _ in range(n)]
    for k, f in zip(box[1], box[2]):
        box_sets[f].add(int((k >> 32) & ((1 << tb) - 1)))
    yy, xx = np.mgrid[0:H, 0:W]
    px, py = xx.ravel() + 0.5, yy.ravel() + 0.5
    for i in range(n):
        assert acc_sets[i] <= box_sets[i], i
        t = min(3.33 ** 2, 2 * np.log(opac[i] * 255.0))
        dx, dy = mean[i, 0] - px, mean[i, 1] - py
        q = conics[i, 0] * dx * dx + 2 * conics[i, 1] * dx * dy + conics[i, 2] * dy * dy
        inside = q < 0.999 * t
        tiles = set(((py[inside] // ts).astype(int) * tw + (px[inside] // ts).astype(int)).tolist())
        assert tiles <= acc_sets[i], (i, tiles - acc_sets[i])


def test_isect_sorted_order_is_key_then_row():
    mean, radii, depths, conics, opac = _ellipse_rows(seed=3)
    depths[:] = 5.0  # force ties on the full key
    tw, th = 13, 10
    unsorted = exact.isect_tiles(mean[None], radii[None], depths[None], 16, tw, th, sort=False,
                                 conics=conics[None], opacities=opac[None])
    srt = exact.isect_tiles(mean[None], radii[None], depths[None], 16, tw, th, sort=True,
                            conics=conics[None], opacities=opac[None])
    order = np.lexsort((unsorted[2], unsorted[1]))
    np.testing.assert_array_equal(srt[1], unsorted[1][order])
    np.testing.assert_array_equal(srt[2], unsorted[2][order])


# --------------------------------------------------------------------------
# Rasterizer
# --------------------------------------------------------------------------
def _raster_inputs(xy, conic, op, color, W=32, H=32, ts=16):
    """Single image: every Gaussian touches every tile, listed front to back."""
    n = len(xy)
    means2d = torch.tensor(xy, dtype=torch.float32)
    conics = torch.tensor(conic, dtype=torch.float32)
    ops = torch.tensor(op, dtype=torch.float32)
    cols = torch.tensor(color, dtype=torch.float32)
    tw, th = W // ts, H // ts
    flatten = torch.arange(n, dtype=torch.int32).repeat(tw * th)
    offsets = (torch.arange(tw * th, dtype=torch.int32) * n).reshape(1, th, tw)
    return means2d, conics, ops, cols, offsets, flatten, W, H, ts


def test_raster_single_gaussian_closed_form():
    xy = [[13.3, 17.8]]
    conic = [[0.05, 0.01, 0.08]]
    m, c, o, col, offs, fl, W, H, ts = _raster_inputs(xy, conic, [0.8], [[0.2, 0.5, 0.9]])
    rc, ra, info = torch_ref.rasterize_to_pixels_ref(m, c, col, o, W, H, ts, offs, fl)
    yy, xx = np.mgrid[0:H, 0:W]
    dx, dy = xy[0][0] - (xx + 0.5), xy[0][1] - (yy + 0.5)
    sig = 0.5 * (conic[0][0] * dx ** 2 + conic[0][2] * dy ** 2) + conic[0][1] * dx * dy
    a = np.minimum(0.99, 0.8 * np.exp(-sig))
    a[a < 1 / 255] = 0
    np.testing.assert_allclose(ra[0, ..., 0].numpy(), a, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(rc[0].numpy(), a[..., None] * np.array([0.2, 0.5, 0.9]),
                               rtol=1e-6, atol=1e-6)


def test_raster_two_gaussians_front_to_back_with_background():
    xy = [[16.0, 16.0], [16.5, 15.5]]
    conic = [[0.02, 0.0, 0.02], [0.03, 0.0, 0.03]]
    m, c, o, col, offs, fl, W, H, ts = _raster_inputs(
        xy, conic, [0.6, 0.9], [[1.0, 0.0, 0.0], [0.0, 1.0, 0.0]])
    bg = torch.tensor([[0.0, 0.0, 1.0]])
    rc, ra, _ = torch_ref.rasterize_to_pixels_ref(m, c, col, o, W, H, ts, offs, fl, backgrounds=bg)
    yy, xx = np.mgrid[0:H, 0:W]

    def alpha(k):
        dx, dy = xy[k][0] - (xx + 0.5), xy[k][1] - (yy + 0.5)
        s = 0.5 * (conic[k][0] * dx ** 2 + conic[k][2] * dy ** 2)
        a = np.minimum(0.99, [0.6, 0.9][k] * np.exp(-s))
        return np.where(a < 1 / 255, 0, a)

    a0, a1 = alpha(0), alpha(1)
    T = (1 - a0) * (1 - a1)
    exp_c = np.stack([a0, a1 * (1 - a0), T], -1)
    np.testing.assert_allclose(rc[0].numpy(), exp_c, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(ra[0, ..., 0].numpy(), 1 - T, rtol=1e-6, atol=1e-6)


def test_raster_termination_is_exclusive():
    # three opaque Gaussians at the same spot: alpha clamps to 0.99, so after
    # the first T = 0.01 and the second would make T = 1e-4 <= threshold.
    xy = [[8.0, 8.0]] * 3
    conic = [[1e-4, 0.0, 1e-4]] * 3
    m, c, o, col, offs, fl, W, H, ts = _raster_inputs(
        xy, conic, [1.0, 1.0, 1.0], [[1.0, 0, 0], [0, 1.0, 0], [0, 0, 1.0]], W=16, H=16)
    rc, ra, info = torch_ref.rasterize_to_pixels_ref(m, c, col, o, W, H, ts, offs, fl)
    np.testing.assert_allclose(ra[0, 8, 8, 0].item(), 0.99, rtol=1e-12)
    np.testing.assert_allclose(rc[0, 8, 8].numpy(), [0.99, 0, 0], rtol=1e-12, atol=1e-12)
    assert info["last_ids"][0, 8, 8] == 0


def test_raster_oracle_grad_matches_finite_differences():
    rng = np.random.default_rng(0)
    n = 6
    xy = rng.uniform(2, 14, (n, 2))
    conic = np.stack([rng.uniform(0.02, 0.2, n), rng.uniform(-0.01, 0.01, n),
                      rng.uniform(0.02, 0.2, n)], -1)
    m, c, o, col, offs, fl, W, H, ts = _raster_inputs(
        xy.tolist(), conic.tolist(), rng.uniform(0.2, 0.9, n).tolist(),
        rng.random((n, 3)).tolist(), W=16, H=16)
    ins = [t.double().requires_grad_() for t in (m, c, col, o)]
    wts = torch.randn(1, 16, 16, 3, dtype=torch.float64)

    def f(mm, cc, cl, oo):
        rc, ra, _ = torch_ref.rasterize_to_pixels_ref(mm, cc, cl, oo, W, H, ts, offs, fl)
        return (rc * wts).sum() + ra.sum()

    assert torch.autograd.gradcheck(f, ins, eps=1e-7, atol=1e-6, rtol=1e-5)


# --------------------------------------------------------------------------
# SH
# --------------------------------------------------------------------------
def test_sh_degree0_closed_form():
    coeffs = torch.randn(5, 1, 3, dtype=torch.float64)
    dirs = torch.randn(5, 3, dtype=torch.float64)
    out = torch_ref.spherical_harmonics_ref(0, dirs, coeffs)
    torch.testing.assert_close(out, 0.2820947917738781 * coeffs[:, 0], rtol=1e-14, atol=0)


def test_sh_basis_is_orthonormal():
    # Gauss-Legendre in cos(theta) x uniform in phi integrates degree <= 8
    # polynomials on the sphere exactly.
    nt, nphi = 24, 48
    xs, ws = np.polynomial.legendre.leggauss(nt)
    phi = (np.arange(nphi) + 0.5) * 2 * np.pi / nphi
    ct, ph = np.meshgrid(xs, phi, indexing="ij")
    st = np.sqrt(1 - ct ** 2)
    d = np.stack([st * np.cos(ph), st * np.sin(ph), ct], -1).reshape(-1, 3)
    w = (ws[:, None] * np.full(nphi, 2 * np.pi / nphi)[None, :]).reshape(-1)
    Y = torch_ref.sh_bases(25, torch.tensor(d)).numpy()
    G = (Y * w[:, None]).T @ Y
    np.testing.assert_allclose(G, np.eye(25), atol=1e-10)


# --------------------------------------------------------------------------
# Adam
# --------------------------------------------------------------------------
def test_adam_first_step_closed_form_and_mask():
    rng = np.random.default_rng(0)
    p = rng.standard_normal((50, 3)).astype(np.float32)
    g = rng.standard_normal((50, 3)).astype(np.float32)
    z = np.zeros_like(p)
    valid = rng.random(50) > 0.3
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-15
    pn, mn, vn = exact.adam(p, g, z, z, valid, lr, b1, b2, eps)
    expect = p - lr * (1 - b1) * g / (np.sqrt(1 - b2) * np.abs(g) + eps)
    np.testing.assert_allclose(pn[valid], expect[valid], rtol=1e-6, atol=6e-8)
    np.testing.assert_array_equal(pn[~valid], p[~valid])
    np.testing.assert_array_equal(mn[~valid], 0)
    np.testing.assert_allclose(mn[valid], (1 - b1) * g[valid], rtol=1e-6)


def test_grad2d_stats_closed_form():
    # gradient (3/640, 4/360) on a 1280x720 image, one camera: the screen-space
    # vector is (3, 4), norm 5; a second camera's row of the same Gaussian
    # (2 cameras: scale doubles) adds 10; culled dense rows add nothing
    grads = torch.tensor([[3 / 640, 4 / 360], [0.0, 0.0], [3 / 640, 4 / 360]])
    g, c = torch_ref.grad2d_stats_ref(grads, torch.tensor([1, 0, 1]), None, 3,
                                      1280, 720, 1)
    assert torch.allclose(g, torch.tensor([0.0, 10.0, 0.0], dtype=torch.float64))
    assert torch.equal(c, torch.tensor([1.0, 2.0, 0.0], dtype=torch.float64))
    g, c = torch_ref.grad2d_stats_ref(grads[:2], torch.tensor([2, 2]), None, 3,
                                      1280, 720, 2)
    assert torch.allclose(g, torch.tensor([0.0, 0.0, 10.0], dtype=torch.float64))
    dense = torch.tensor([[[3 / 640, 4 / 360], [1.0, 1.0]]])
    radii = torch.tensor([[[2, 3], [0, 5]]], dtype=torch.int32)
    g, c = torch_ref.grad2d_stats_ref(dense, None, radii, 2, 1280, 720, 1)
    assert torch.allclose(g, torch.tensor([5.0, 0.0], dtype=torch.float64))
    assert torch.equal(c, torch.tensor([1.0, 0.0], dtype=torch.float64))


def test_rasterize_to_indices_oracle_single_gaussian_closed_form():
    # one isotropic Gaussian (conic 1/s^2 I) centred in a 16x16 tile, opacity
    # 0.8, full transmittance: the pairs are exactly the pixels with
    # sigma = |d|^2 / (2 s^2) <= ln(255 * 0.8), in pixel order
    s2 = 9.0
    m2 = np.array([[8.0, 8.0]], np.float32)
    con = np.array([[1 / s2, 0.0, 1 / s2]], np.float32)
    op = np.array([0.8], np.float32)
    offs = np.zeros((1, 1, 1), np.int32)
    gids, pids = exact.rasterize_to_indices(0, 10 ** 9, np.ones((1, 16, 16), np.float32),
                                            m2, con, op, 16, 16, 16, offs,
                                            np.zeros(1, np.int32), 1)
    yy, xx = np.mgrid[0:16, 0:16]
    d2 = (xx + 0.5 - 8.0) ** 2 + (yy + 0.5 - 8.0) ** 2
    expect = np.nonzero((d2 / (2 * s2) <= math.log(255 * 0.8)).ravel())[0]
    np.testing.assert_array_equal(pids, expect)
    assert (gids == 0).all()
    # a pixel whose transmittance is already at the cutoff takes nothing
    T = np.ones((1, 16, 16), np.float32)
    T[0, 8, 8] = 1e-4
    _, pids2 = exact.rasterize_to_indices(0, 10 ** 9, T, m2, con, op, 16, 16, 16, offs,
                                          np.zeros(1, np.int32), 1)
    assert 8 * 16 + 8 not in set(pids2.tolist())
    assert len(pids2) == len(pids) - 1
    # batches past the tile's range leave every pixel empty
    g3, _ = exact.rasterize_to_indices(1, 10 ** 9, np.ones((1, 16, 16), np.float32),
                                       m2, con, op, 16, 16, 16, offs,
                                       np.zeros(1, np.int32), 1)
    assert g3.size == 0


def test_rasterize_to_indices_oracle_agrees_with_compositing_oracle():
    # full range from T = 1: every pixel's last pair is the forward oracle's
    # last composited Gaussian, and pixels with no pair have alpha 0
    from tests._util import projected_2d
    d = projected_2d(seed=5, N=400, C=1, W=48, H=40)
    N = d["means2d"].shape[-2]
    gids, pids = exact.rasterize_to_indices(
        0, 10 ** 9, np.ones((1, d["H"], d["W"]), np.float32), d["means2d"].numpy(),
        d["conics"].numpy(), d["opacities"].numpy(), d["W"], d["H"], d["tile"],
        d["offsets"].numpy(), d["flatten_ids"].numpy(), N)
    _, ra, info = torch_ref.rasterize_to_pixels_ref(
        d["means2d"].double(), d["conics"].double(), d["colors"].double(),
        d["opacities"].double(), d["W"], d["H"], d["tile"], d["offsets"],
        d["flatten_ids"])
    fl = d["flatten_ids"].numpy()
    last = info["last_ids"].reshape(-1)
    alpha = ra.detach().numpy().reshape(-1)
    has = np.zeros(alpha.size, bool)
    has[pids] = True
    np.testing.assert_array_equal(has, alpha > 0)
    assert pids.size > 1000
    ends = np.r_[np.nonzero(np.diff(pids))[0], pids.size - 1]
    np.testing.assert_array_equal(gids[ends], fl[last[pids[ends]]] % N)
    assert (np.diff(pids) >= 0).all()


def test_precision_oracle_is_the_covariance_inverse():
    g = torch.Generator().manual_seed(0)
    q = torch.randn(64, 4, generator=g, dtype=torch.float64)
    s = torch.rand(64, 3, generator=g, dtype=torch.float64) + 0.2
    C = torch_ref.quat_scale_to_covar(q, s)
    R = torch_ref.quat_to_rotmat(q)
    P = R @ torch.diag_embed(1.0 / s ** 2) @ R.transpose(-1, -2)
    torch.testing.assert_close(C @ P, torch.eye(3, dtype=torch.float64).expand(64, 3, 3))
