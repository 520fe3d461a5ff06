"""EWA projection on the GPU against the host oracles.

Forward: every output bit-exact against the C restatement (exact_ref.c), for
the dense and packed layouts, quats/scales and covars inputs, pinhole and
ortho cameras, batch dims, opacity-aware radii and compensation.
Backward: against autograd of the float64 PyTorch restatement, within
rtol 1e-4 / atol 1e-5 at the float32 floor that the same restatement
evaluated in float32 measures (tests/_util.py:assert_grad_close)."""

import numpy as np
import pytest
import torch

from oracle import exact, torch_ref
from tests._util import DEV, assert_close, assert_grad_close, small_scene

pytestmark = pytest.mark.gpu


def _bits(a):
    a = a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else a
    return np.ascontiguousarray(a).view(np.uint32 if a.dtype == np.float32 else a.dtype)


def _covars6(quats, scales):
    S = torch_ref.quat_scale_to_covar(quats.double(), scales.double()).float()
    return S[..., [0, 0, 0, 1, 1, 2], [0, 1, 2, 1, 2, 2]].contiguous()


@pytest.mark.parametrize("camera_model", ["pinhole", "ortho"])
@pytest.mark.parametrize("use_covars", [False, True])
@pytest.mark.parametrize("with_opacity,calc_comp", [(False, False), (True, False), (True, True)])
def test_fused_fwd_bitexact(camera_model, use_covars, with_opacity, calc_comp):
    from gsplat_amd.cuda import _ops
    means, quats, scales, opac, vm, K, W, H = small_scene(seed=1, N=3000, C=3)
    if camera_model == "ortho":
        K = K.clone()
        K[:, 0, 0] = 30.0
        K[:, 1, 1] = 30.0
    covars = _covars6(quats, scales) if use_covars else None
    cm = {"pinhole": 0, "ortho": 1}[camera_model]
    op = opac if with_opacity else None
    ex = exact.projection_fwd(means.numpy(), None if covars is None else covars.numpy(),
                              None if use_covars else quats.numpy(),
                              None if use_covars else scales.numpy(),
                              None if op is None else op.numpy(), vm.numpy(), K.numpy(),
                              W, H, 0.3, 0.01, 1e10, 0.0, calc_comp, cm)
    d = lambda t: None if t is None else t.to(DEV)
    radii, m2, dep, con, comp = _ops.projection_ewa_3dgs_fused_fwd(
        d(means), d(covars), None if use_covars else d(quats),
        None if use_covars else d(scales), d(op), d(vm), d(K), W, H, 0.3, 0.01,
        1e10, 0.0, calc_comp, cm)
    assert ex["valid"].sum() > 100
    np.testing.assert_array_equal(radii.cpu().numpy(), ex["radii"])
    np.testing.assert_array_equal(_bits(m2), _bits(ex["means2d"]))
    np.testing.assert_array_equal(_bits(dep), _bits(ex["depths"]))
    np.testing.assert_array_equal(_bits(con), _bits(ex["conics"]))
    if calc_comp:
        np.testing.assert_array_equal(_bits(comp), _bits(ex["compensations"]))


@pytest.mark.parametrize("batch_dims", [(), (2,)])
def test_packed_fwd_bitexact(batch_dims):
    from gsplat_amd.cuda import _ops
    means, quats, scales, opac, vm, K, W, H = small_scene(seed=2, N=5000, C=3)
    if batch_dims:
        means = torch.stack([means, means.flip(0)])
        quats = torch.stack([quats, quats.flip(0)])
        scales = torch.stack([scales, scales.flip(0)])
        opac = torch.stack([opac, opac.flip(0)])
        vm = torch.stack([vm, vm.flip(0)])
        K = torch.stack([K, K])
    B = int(np.prod(batch_dims)) if batch_dims else 1
    C, N = vm.shape[-3], means.shape[-2]
    ex = exact.projection_fwd(means.numpy(), None, quats.numpy(), scales.numpy(),
                              opac.numpy(), vm.numpy(), K.numpy(), W, H, 0.3, 0.01,
                              1e10, 0.0, True, 0)
    pk = exact.pack_projection(ex, B, C, N)
    out = _ops.projection_ewa_3dgs_packed_fwd(
        means.to(DEV), None, quats.to(DEV), scales.to(DEV), opac.to(DEV), vm.to(DEV),
        K.to(DEV), W, H, 0.3, 0.01, 1e10, 0.0, True, 0)
    names = ["indptr", "batch_ids", "camera_ids", "gaussian_ids", "radii", "means2d",
             "depths", "conics", "compensations"]
    for name, got in zip(names, out):
        want = pk[name]
        assert got.shape[0] == want.shape[0], name
        np.testing.assert_array_equal(_bits(got), _bits(want), err_msg=name)


def _grad_check(packed, calc_comp, use_covars=False, viewmat_grad=True, C=2):
    from gsplat_amd.cuda._wrapper import fully_fused_projection
    means, quats, scales, opac, vm, K, W, H = small_scene(seed=3, N=1500, C=C)
    covars = _covars6(quats, scales) if use_covars else None
    N = means.shape[0]
    ex = exact.projection_fwd(means.numpy(), None if covars is None else covars.numpy(),
                              None if use_covars else quats.numpy(),
                              None if use_covars else scales.numpy(), opac.numpy(),
                              vm.numpy(), K.numpy(), W, H, 0.3, 0.01, 1e10, 0.0,
                              calc_comp, 0)
    valid = torch.from_numpy(ex["valid"])
    g = torch.Generator().manual_seed(7)
    w_m = torch.randn(C, N, 2, generator=g)
    w_c = torch.randn(C, N, 3, generator=g)
    w_d = torch.randn(C, N, generator=g)
    w_p = torch.randn(C, N, generator=g)

    # GPU
    leaves = {
        "means": means.clone().to(DEV).requires_grad_(),
        "viewmats": vm.clone().to(DEV).requires_grad_(viewmat_grad),
    }
    if use_covars:
        leaves["covars"] = covars.clone().to(DEV).requires_grad_()
    else:
        leaves["quats"] = quats.clone().to(DEV).requires_grad_()
        leaves["scales"] = scales.clone().to(DEV).requires_grad_()
    out = fully_fused_projection(
        leaves["means"], leaves.get("covars"), leaves.get("quats"), leaves.get("scales"),
        leaves["viewmats"], K.to(DEV), W, H, packed=packed, calc_compensations=calc_comp,
        opacities=opac.to(DEV))
    if packed:
        b, c, gid, indptr, radii, m2, dep, con, comp = out
        rows = (c * N + gid)
        wm, wc, wd, wp = (w.reshape((C * N,) + w.shape[2:]).to(DEV)[rows]
                          for w in (w_m, w_c, w_d, w_p))
        loss = (m2 * wm).sum() + (con * wc).sum() + (dep * wd).sum()
        if calc_comp:
            loss = loss + (comp * wp).sum()
    else:
        radii, m2, dep, con, comp = out
        vmask = valid.to(DEV)
        loss = (m2 * w_m.to(DEV))[vmask].sum() + (con * w_c.to(DEV))[vmask].sum() + \
            (dep * w_d.to(DEV))[vmask].sum()
        if calc_comp:
            loss = loss + (comp * w_p.to(DEV))[vmask].sum()
    loss.backward()

    # oracle (float64 autograd)
    ref_leaves = {k: (v.detach().cpu().double().requires_grad_(v.requires_grad))
                  for k, v in leaves.items()}
    t = torch_ref.projection_ref(ref_leaves["means"], ref_leaves.get("covars"),
                                 ref_leaves.get("quats"), ref_leaves.get("scales"),
                                 ref_leaves["viewmats"], K.double(), W, H,
                                 calc_compensations=calc_comp)
    v = valid
    rl = (t["means2d"] * w_m.double())[v].sum() + (t["conics"] * w_c.double())[v].sum() + \
        (t["depths"] * w_d.double())[v].sum()
    if calc_comp:
        rl = rl + (t["compensations"] * w_p.double())[v].sum()
    rl.backward()
    # the same restatement in float32: its error measures the fp32 floor
    l32 = {k: (v.detach().cpu().float().requires_grad_(v.requires_grad))
           for k, v in leaves.items()}
    t32 = torch_ref.projection_ref(l32["means"], l32.get("covars"), l32.get("quats"),
                                   l32.get("scales"), l32["viewmats"], K, W, H,
                                   calc_compensations=calc_comp)
    r32 = (t32["means2d"] * w_m)[v].sum() + (t32["conics"] * w_c)[v].sum() + \
        (t32["depths"] * w_d)[v].sum()
    if calc_comp:
        r32 = r32 + (t32["compensations"] * w_p)[v].sum()
    r32.backward()
    for k in leaves:
        if not leaves[k].requires_grad:
            continue
        assert_grad_close(leaves[k].grad, ref_leaves[k].grad, l32[k].grad,
                          rtol=1e-4, atol=1e-5, name=f"d{k}")


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("calc_comp", [False, True])
def test_projection_bwd_vs_autograd(packed, calc_comp):
    _grad_check(packed, calc_comp)


def test_projection_bwd_covars_single_camera():
    _grad_check(False, False, use_covars=True, C=1)
    _grad_check(True, False, use_covars=True, C=1)


def test_packed_sparse_grad_matches_dense():
    from gsplat_amd.cuda._wrapper import fully_fused_projection
    means, quats, scales, opac, vm, K, W, H = small_scene(seed=4, N=1000, C=1)
    outs = []
    for sparse in (False, True):
        leaves = [t.clone().to(DEV).requires_grad_() for t in (means, quats, scales)]
        b, c, gid, indptr, radii, m2, dep, con, comp = fully_fused_projection(
            leaves[0], None, leaves[1], leaves[2], vm.to(DEV), K.to(DEV), W, H,
            packed=True, sparse_grad=sparse)
        (m2.sum() + con.sum() * 3 + dep.sum()).backward()
        outs.append([l.grad.to_dense() if l.grad.is_sparse else l.grad for l in leaves])
    # the sparse rows come from the row-driven kernel, the dense gradient from
    # the Gaussian-driven one: same math, compiled (and contracted into FMAs)
    # separately, so they agree to float32 rounding, not bit for bit
    for a, b in zip(*outs):
        assert_close(a, b, 1e-4, 1e-5, "sparse vs dense")


@pytest.mark.parametrize("C,use_covars", [(1, False), (3, False), (2, True)])
def test_packed_bwd_rows_matches_row_scatter(C, use_covars):
    """The Gaussian-driven backward over the row map equals the row-driven
    packed backward (atomics into zero-filled outputs) up to summation order;
    an absent depth gradient equals a zero one."""
    from gsplat_amd.cuda import _ops
    means, quats, scales, opac, vm, K, W, H = small_scene(seed=9, N=3000, C=C)
    covars = _covars6(quats, scales) if use_covars else None
    d = lambda t: None if t is None else t.to(DEV)
    q, s = (None, None) if use_covars else (d(quats), d(scales))
    out = _ops.projection_packed_fwd_with_row_map(
        d(means), d(covars), q, s, d(opac), d(vm), d(K), W, H, 0.3, 0.01, 1e10, 0.0,
        False, 0)
    indptr, b, c, g, radii, m2, dep, con, comp, row_of = out
    nnz = m2.shape[0]
    gen = torch.Generator().manual_seed(C)
    vm2 = torch.randn(nnz, 2, generator=gen).to(DEV)
    vcon = torch.randn(nnz, 3, generator=gen).to(DEV)
    vdep = torch.randn(nnz, generator=gen).to(DEV)
    ref = _ops.projection_ewa_3dgs_packed_bwd(
        d(means), d(covars), q, s, d(vm), d(K), W, H, 0.3, 0, b, c, g, con, None,
        vm2, vdep, vcon, None, True, False)
    got = _ops.projection_packed_bwd_rows(
        d(means), d(covars), q, s, d(vm), d(K), W, H, 0.3, 0, row_of, con, None,
        vm2, vdep, vcon, None, True)
    # two float32 sums of the same per-camera terms in different orders
    # (cancellation between cameras makes element-wise relative error
    # meaningless): held norm-wise; both are checked against the float64
    # restatement elementwise by test_projection_bwd_vs_autograd
    for name, x, y in zip(("means", "covars", "quats", "scales", "viewmats"), got, ref):
        if y is None:
            assert x is None
            continue
        err = (x - y).abs().max().item()
        assert err <= 1e-4 * y.abs().max().item() + 1e-5, (name, err)
    # v_depths = None is a zero depth gradient
    got0 = _ops.projection_packed_bwd_rows(
        d(means), d(covars), q, s, d(vm), d(K), W, H, 0.3, 0, row_of, con, None,
        vm2, None, vcon, None, False)
    ref0 = _ops.projection_packed_bwd_rows(
        d(means), d(covars), q, s, d(vm), d(K), W, H, 0.3, 0, row_of, con, None,
        vm2, torch.zeros_like(vdep), vcon, None, False)
    for x, y in zip(got0, ref0):
        if y is not None:
            assert torch.equal(x, y)


@pytest.mark.parametrize("calc_comp", [False, True])
def test_packed_sparse_grad_rows_match_per_row_autograd(calc_comp):
    """sparse_grad=True (ProjectionEWA3DGSPacked.cu:578-611,
    _wrapper.py:2258-2305): the op returns one gradient row per packed row,
    indexed by gaussian_ids and not summed over cameras.  Each row is held to
    the float64 autograd gradient of that row's own outputs alone: the
    restatement is run per camera on a copy of the Gaussians of that camera's
    rows, so every leaf row sees exactly one packed row."""
    from gsplat_amd.cuda import _ops
    C = 2
    means, quats, scales, opac, vm, K, W, H = small_scene(seed=12, N=2500, C=C)
    d = lambda t: t.to(DEV)
    out = _ops.projection_ewa_3dgs_packed_fwd(
        d(means), None, d(quats), d(scales), d(opac), d(vm), d(K), W, H, 0.3, 0.01,
        1e10, 0.0, calc_comp, 0)
    indptr, b, cam, gid, radii, m2, dep, con, comp = out
    nnz = m2.shape[0]
    g = torch.Generator().manual_seed(13)
    v_m2 = torch.randn(nnz, 2, generator=g)
    v_con = torch.randn(nnz, 3, generator=g)
    v_dep = torch.randn(nnz, generator=g)
    v_comp = torch.randn(nnz, generator=g) if calc_comp else None
    v_means, _, v_quats, v_scales, _ = _ops.projection_ewa_3dgs_packed_bwd(
        d(means), None, d(quats), d(scales), d(vm), d(K), W, H, 0.3, 0, b, cam, gid,
        con, comp, d(v_m2), d(v_dep), d(v_con),
        None if v_comp is None else d(v_comp), False, True)
    assert v_means.shape == (nnz, 3) and v_quats.shape == (nnz, 4)

    cam_np, gid_np = cam.cpu().numpy(), gid.cpu().numpy()
    got = {"means": v_means.cpu(), "quats": v_quats.cpu(), "scales": v_scales.cpu()}
    ref = {k: torch.zeros(nnz, t.shape[1], dtype=torch.float64) for k, t in got.items()}
    ref32 = {k: torch.zeros(nnz, t.shape[1], dtype=torch.float64) for k, t in got.items()}
    for dtype, dst in ((torch.float64, ref), (torch.float32, ref32)):
        for c in range(C):
            rows = np.nonzero(cam_np == c)[0]
            gi = torch.from_numpy(gid_np[rows])
            leaves = {k: src[gi].to(dtype).clone().requires_grad_()
                      for k, src in (("means", means), ("quats", quats), ("scales", scales))}
            t = torch_ref.projection_ref(leaves["means"], None, leaves["quats"],
                                         leaves["scales"], vm[c:c + 1].to(dtype),
                                         K[c:c + 1].to(dtype), W, H,
                                         calc_compensations=calc_comp)
            r = torch.from_numpy(rows)
            loss = (t["means2d"][0] * v_m2[r].to(dtype)).sum() + \
                (t["conics"][0] * v_con[r].to(dtype)).sum() + \
                (t["depths"][0] * v_dep[r].to(dtype)).sum()
            if calc_comp:
                loss = loss + (t["compensations"][0] * v_comp[r].to(dtype)).sum()
            loss.backward()
            for k in dst:
                dst[k][r] = leaves[k].grad.double()
    for k in got:
        print(assert_grad_close(got[k], ref[k], ref32[k], 1e-4, 1e-5, f"sparse d{k}"))
