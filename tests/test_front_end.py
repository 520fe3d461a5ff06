"""rasterization()'s packed front end in one autograd node (projection, row
opacities and row colours; rendering.py:256-873) against the separate nodes
it replaces: ``_FullyFusedProjectionPacked`` + ``_PackedRowsGather`` (the
reference's opacities[batch_ids, gaussian_ids]) + ``_PackedSphericalHarmonics``
or a colour gather.  Those separate nodes are themselves pinned against the
oracle (test_projection.py, test_packed_rows.py).  Same kernels on the same
inputs, so the forward outputs must agree bit for bit.  The gradients use the
same kernels too: only v_means adds the SH term inside the projection pass
instead of in autograd (one float addition either way, a + b == b + a), and
v_opacities sums a Gaussian's rows over the cameras in the same order.  So
the gradients are also required to agree exactly."""

import math

import pytest
import torch

from tests._util import DEV, small_scene

pytestmark = pytest.mark.gpu


def _covars_triu(quats, scales):
    q = torch.nn.functional.normalize(quats.double(), dim=-1)
    w, x, y, z = q.unbind(-1)
    R = torch.stack([
        1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
        2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
        2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)],
        -1).reshape(*q.shape[:-1], 3, 3)
    M = R * scales.double()[..., None, :]
    S = M @ M.transpose(-1, -2)
    i, j = [0, 0, 0, 1, 1, 2], [0, 1, 2, 1, 2, 2]
    return S[..., i, j].float()


def _inputs(seed, N, C, batch, sh_degree, D, covars):
    means, quats, scales, opac, vm, K, W, H = small_scene(seed=seed, N=N, C=C)
    g = torch.Generator().manual_seed(seed + 7)
    if sh_degree is None:
        feats = torch.rand(N, D, generator=g)
    else:
        feats = torch.randn(N, (sh_degree + 1) ** 2, 3, generator=g) * 0.3
    if batch:
        # a second batch entry: the same cameras, Gaussians moved a little
        def two(t, eps):
            return torch.stack([t, t + eps * torch.randn(t.shape, generator=g)])
        means, quats, scales = two(means, 0.05), two(quats, 0.05), two(scales, 0.0)
        opac, feats = two(opac, 0.0), two(feats, 0.05)
        vm, K = torch.stack([vm, vm]), torch.stack([K, K])
    leaves = {"means": means, "opac": opac, "feats": feats}
    if covars:
        leaves["covars"] = _covars_triu(quats, scales)
    else:
        leaves["quats"], leaves["scales"] = quats, scales
    leaves = {k: v.to(DEV).contiguous() for k, v in leaves.items()}
    return leaves, vm.to(DEV).contiguous(), K.to(DEV).contiguous(), W, H


def _run(fused, leaves, vm, K, W, H, sh_degree, antialiased, weights):
    from gsplat_amd.cuda._wrapper import (_FullyFusedProjectionPacked,
                                          _PackedFrontEnd, _PackedRowsGather,
                                          _PackedSphericalHarmonics)
    lv = {k: v.clone().requires_grad_() for k, v in leaves.items()}
    covars, quats, scales = lv.get("covars"), lv.get("quats"), lv.get("scales")
    means, opac, feats = lv["means"], lv["opac"], lv["feats"]
    args = (W, H, 0.3, 0.01, 1e10, 0.0)
    if fused:
        out = _PackedFrontEnd.apply(means, covars, quats, scales, opac, feats, vm, K,
                                    *args, antialiased, "pinhole", sh_degree)
        (b, c, gid, indptr, radii, m2, dep, con, comp, row_of, r_op, r_col) = out
    else:
        (b, c, gid, indptr, radii, m2, dep, con, comp,
         row_of) = _FullyFusedProjectionPacked.apply(
            means, covars, quats, scales, vm, K, *args, False, antialiased,
            "pinhole", opac)
        nnz = m2.shape[0]
        Bn, N, C = math.prod(means.shape[:-2]), means.shape[-2], vm.shape[-3]
        r_op = _PackedRowsGather.apply(opac.reshape(Bn, N, 1), row_of, C,
                                       nnz).reshape(nnz)
        if sh_degree is None:
            r_col = _PackedRowsGather.apply(feats.reshape(Bn, N, -1), row_of, C, nnz)
        else:
            r_col = _PackedSphericalHarmonics.apply(
                sh_degree, means.reshape(Bn, N, 3),
                feats.reshape(Bn, N, *feats.shape[-2:]), vm.reshape(Bn, C, 4, 4),
                row_of, nnz)
    outs = {"batch_ids": b, "camera_ids": c, "gaussian_ids": gid, "indptr": indptr,
            "radii": radii, "means2d": m2, "depths": dep, "conics": con,
            "row_of": row_of, "row_opacities": r_op, "row_colors": r_col}
    if comp is not None:
        outs["compensations"] = comp
    nnz = m2.shape[0]
    loss = ((m2 * weights["m2"][:nnz]).sum() + (con * weights["con"][:nnz]).sum()
            + (dep * weights["dep"][:nnz]).sum() + (r_op * weights["op"][:nnz]).sum()
            + (r_col * weights["col"][:nnz, :r_col.shape[1]]).sum())
    if comp is not None:
        loss = loss + (comp * weights["op"][:nnz]).sum()
    loss.backward()
    return outs, {k: v.grad for k, v in lv.items()}


@pytest.mark.parametrize("case", [
    dict(C=1, sh_degree=3),
    dict(C=3, sh_degree=2),
    dict(C=2, sh_degree=None, D=4),
    dict(C=1, sh_degree=3, antialiased=True),
    dict(C=2, sh_degree=1, batch=True),
    dict(C=2, sh_degree=3, covars=True),
])
def test_front_end_matches_separate_nodes(case):
    C = case["C"]
    sh_degree = case.get("sh_degree")
    leaves, vm, K, W, H = _inputs(3 + C, 3000, C, case.get("batch", False), sh_degree,
                                  case.get("D", 3), case.get("covars", False))
    cap = math.prod(leaves["means"].shape[:-1]) * C
    g = torch.Generator().manual_seed(11)
    weights = {k: torch.randn(cap, n, generator=g).squeeze(-1).to(DEV)
               for k, n in (("m2", 2), ("con", 3), ("dep", 1), ("op", 1), ("col", 4))}
    antialiased = case.get("antialiased", False)
    of, gf = _run(True, leaves, vm, K, W, H, sh_degree, antialiased, weights)
    os_, gs_ = _run(False, leaves, vm, K, W, H, sh_degree, antialiased, weights)
    assert of.keys() == os_.keys()
    assert of["means2d"].shape[0] > 100
    for k in of:
        assert torch.equal(of[k], os_[k]), k
    for k in gf:
        assert gf[k] is not None and gs_[k] is not None, k
        assert torch.equal(gf[k], gs_[k]), (k, (gf[k] - gs_[k]).abs().max().item())


def test_queued_emission_matches_exact_and_falls_back():
    """rasterization() three times on one scene: the first call emits the
    intersections with the count read on the host, the second queues the
    emission with the count read on the device (capacity from the first
    count), the third is given a capacity below the count and must fall back
    to the exact emission.  All three give the same intersections and
    renders."""
    import gsplat_amd as gs
    from gsplat_amd.cuda import _ops

    means, quats, scales, opac, vm, K, W, H = small_scene(seed=5, N=6000, C=1, W=320,
                                                          H=240)
    g = torch.Generator().manual_seed(9)
    coeffs = (torch.randn(6000, 16, 3, generator=g) * 0.3).to(DEV)
    args = [t.to(DEV) for t in (means, quats, scales, opac)]
    names = []
    real_call = _ops.call

    def spy(name, *a):
        names.append(name)
        return real_call(name, *a)

    def render():
        names.clear()
        rc, ra, meta = gs.rasterization(*args, coeffs, vm.to(DEV), K.to(DEV), W, H,
                                        sh_degree=3, packed=True)
        return rc, ra, meta, list(names)

    dev = torch.device(DEV)
    _ops._ISECT_LAST.pop(dev.index if dev.index is not None else 0, None)
    _ops._ISECT_LAST.pop(torch.cuda.current_device(), None)
    _ops.call = spy
    try:
        out = [render()]
        n = out[0][2]["isect_ids"].numel()
        assert n > 5000
        out.append(render())
        _ops._ISECT_LAST[torch.cuda.current_device()] = 10  # capacity 4107 < n
        out.append(render())
    finally:
        _ops.call = real_call
    assert "gsplat_isect_emit_tiles_dev" not in out[0][3]
    assert "gsplat_isect_emit_tiles_dev" in out[1][3]
    assert "gsplat_isect_emit_tiles" not in out[1][3]
    assert "gsplat_isect_emit_tiles_dev" in out[2][3]
    assert "gsplat_isect_emit_tiles" in out[2][3]
    for rc, ra, meta, _ in out[1:]:
        for k in ("isect_ids", "flatten_ids", "isect_offsets"):
            assert torch.equal(meta[k], out[0][2][k]), k
        assert torch.equal(rc, out[0][0])
        assert torch.equal(ra, out[0][1])


@pytest.mark.parametrize("packed", [True, False])
def test_rasterization_with_every_gaussian_culled(packed):
    """Every Gaussian behind the camera: no visible rows and no intersections
    (the front end's count is 0, the intersection stages are skipped).  The
    image is the background, alpha 0, and every gradient is zero (the
    reference's behaviour: nothing composites)."""
    import gsplat_amd as gs
    from gsplat_amd.cuda import _ops

    means, quats, scales, opac, vm, K, W, H = small_scene(seed=2, N=500, C=1)
    means = means.clone()
    means[:, 2] = means[:, 2] - 100.0  # z of every mean behind the camera
    g = torch.Generator().manual_seed(3)
    coeffs = (torch.randn(500, 4, 3, generator=g) * 0.3).to(DEV).requires_grad_()
    leaves = [t.to(DEV).requires_grad_() for t in (means, quats, scales, opac)]
    # backgrounds [C, D] only on the dense path: packed rasterize_to_pixels
    # takes [D] (its image dims are empty), as in the reference
    # (_wrapper.py:868-885)
    bg = None if packed else torch.tensor([[0.2, 0.4, 0.6]], device=DEV)
    for _ in range(2):  # the second call also sees the previous intersection count
        rc, ra, meta = gs.rasterization(*leaves, coeffs, vm.to(DEV), K.to(DEV), W, H,
                                        sh_degree=1, packed=packed, backgrounds=bg)
        if packed:
            assert meta["means2d"].shape[0] == 0
        assert meta["isect_ids"].numel() == 0
        expect = torch.zeros(3, device=DEV) if bg is None else bg.reshape(3)
        assert torch.equal(rc, expect.expand_as(rc))
        assert torch.equal(ra, torch.zeros_like(ra))
        (rc.sum() + ra.sum()).backward()
        for t in leaves + [coeffs]:
            assert t.grad is not None and torch.count_nonzero(t.grad) == 0
            t.grad = None
    _ops._ISECT_LAST.clear()
