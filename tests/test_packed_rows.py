"""Per-Gaussian gathers of the packed path (rendering.py:95-213, 782,
845-873) driven by the projection's inverse map ``row_of``: against plain
indexing (gather: bit-exact), a float64 index_add (scatter), and autograd of
the float64 SH restatement of gather + normalize + SH + clamp_min(+0.5, 0)
(fused SH rows)."""

import numpy as np
import pytest
import torch

from oracle import torch_ref
from tests._util import DEV, assert_close, assert_grad_close, small_scene

pytestmark = pytest.mark.gpu


def _packed(seed, N, C):
    from gsplat_amd.cuda import _ops
    means, quats, scales, opac, vm, K, W, H = small_scene(seed=seed, N=N, C=C)
    out = _ops.projection_packed_fwd_with_row_map(
        means.to(DEV), None, quats.to(DEV), scales.to(DEV), opac.to(DEV),
        vm.to(DEV), K.to(DEV), W, H, 0.3, 0.01, 1e10, 0.0, False, 0)
    indptr, b, c, g, radii, m2, dep, con, comp, row_of = out
    return means, vm, b.cpu(), c.cpu(), g.cpu(), row_of, m2.shape[0]


@pytest.mark.parametrize("C", [1, 3])
def test_row_map_is_the_inverse_of_the_ids(C):
    means, vm, b, c, g, row_of, nnz = _packed(1, 2000, C)
    ro = row_of.cpu().numpy().reshape(C, -1)
    N = means.shape[0]
    expect = np.full((C, N), -1, np.int64)
    expect[c.numpy(), g.numpy()] = np.arange(nnz)
    np.testing.assert_array_equal(ro, expect)


@pytest.mark.parametrize("C,F", [(1, 1), (3, 1), (3, 3), (2, 5)])
def test_rows_gather_and_scatter(C, F):
    from gsplat_amd.cuda import _ops
    means, vm, b, c, g, row_of, nnz = _packed(2, 3000, C)
    N = means.shape[0]
    gen = torch.Generator().manual_seed(5)
    src = torch.randn(1, N, F, generator=gen)
    out = _ops.rows_gather(src.to(DEV), row_of, C, nnz)
    assert torch.equal(out.cpu(), src[0, g])
    v_out = torch.randn(nnz, F, generator=gen)
    v_src = _ops.rows_scatter_sum(v_out.to(DEV), row_of, 1, C, N)
    ref = torch.zeros(N, F, dtype=torch.float64).index_add_(0, g, v_out.double())
    assert_close(v_src.cpu()[0], ref, 1e-6, 1e-7, "v_src")
    # Gaussians visible nowhere get an explicit zero row
    seen = torch.zeros(N, dtype=torch.bool)
    seen[g] = True
    assert bool((v_src.cpu()[0][~seen] == 0).all())


@pytest.mark.parametrize("degree,C", [(0, 1), (1, 3), (2, 2), (3, 1), (3, 3), (4, 2)])
def test_sh_rows_fwd_bwd(degree, C):
    from gsplat_amd.cuda._wrapper import _PackedSphericalHarmonics
    from gsplat_amd.rendering import viewmat_to_camera_position
    means, vm, b, c, g, row_of, nnz = _packed(3 + degree, 2500, C)
    N = means.shape[0]
    K = (degree + 1) ** 2 + (3 if degree == 2 else 0)  # one case with extra bands
    gen = torch.Generator().manual_seed(degree)
    coeffs = torch.randn(N, K, 3, generator=gen) * 0.4
    campos = viewmat_to_camera_position(vm)
    v_col = torch.randn(nnz, 3, generator=gen)

    gm = means.clone().to(DEV).requires_grad_()
    gc = coeffs.clone().to(DEV).requires_grad_()
    col = _PackedSphericalHarmonics.apply(degree, gm[None], gc[None],
                                          vm[None].to(DEV), row_of, nnz)
    (col * v_col.to(DEV)).sum().backward()

    def ref(dtype):
        m = means.to(dtype).requires_grad_()
        cf = coeffs.to(dtype).requires_grad_()
        dirs = m[g] - campos.to(dtype)[c]
        out = torch.clamp_min(
            torch_ref.spherical_harmonics_ref(degree, dirs, cf[g]) + 0.5, 0.0)
        (out * v_col.to(dtype)).sum().backward()
        # degree 0 does not depend on the direction: no graph to the means
        mg = m.grad if m.grad is not None else torch.zeros_like(m)
        return out, mg, cf.grad

    r64, m64, c64 = ref(torch.float64)
    r32, m32, c32 = ref(torch.float32)
    assert_close(col.cpu(), r64.detach(), 1e-4, 1e-5, "colors")
    print(assert_grad_close(gc.grad, c64, c32, 1e-4, 1e-5, "v_coeffs"))
    print(assert_grad_close(gm.grad, m64, m32, 1e-4, 1e-5, "v_means"))


@pytest.mark.parametrize("degree,C", [(3, 1), (1, 3), (0, 2), (4, 1)])
def test_fused_colours_and_tile_counts_match_the_separate_launches(degree, C):
    """gsplat_sh_rows_fwd_isect_count + gsplat_isect_row_starts against
    gsplat_sh_rows_fwd and gsplat_isect_prepare_rows on the same packed rows:
    colours, tile counts, row starts, the intersection count and the sweep
    records equal bit for bit; the row count is read from indptr[C] on the
    device, and the capacity-sized buffers past it are not written."""
    import math

    from gsplat_amd._lib import call, ptr, query
    from gsplat_amd.cuda import _ops
    means, quats, scales, opac, vm, K, W, H = small_scene(seed=40 + degree, N=3000, C=C)
    N = means.shape[0]
    gen = torch.Generator().manual_seed(7)
    coeffs = torch.randn(1, N, (degree + 1) ** 2, 3, generator=gen).to(DEV)
    md, vmd = means.to(DEV)[None], vm.to(DEV)[None]
    out = _ops.projection_packed_fwd_with_row_map(
        means.to(DEV), None, quats.to(DEV), scales.to(DEV), opac.to(DEV),
        vm.to(DEV), K.to(DEV), W, H, 0.3, 0.01, 1e10, 0.0, False, 0)
    indptr, b, c, g, radii, m2, dep, con, comp, row_of = out
    nnz = m2.shape[0]
    cap = C * N
    assert 0 < nnz < cap
    row_opac = opac.to(DEV)[g]
    ts = 16
    tw, th = math.ceil(W / ts), math.ceil(H / ts)
    img = c if C > 1 else None

    # separate launches
    colors_ref = _ops.sh_rows_fwd(degree, md, vmd, coeffs, row_of, nnz)
    state = _ops.isect_prepare_sorted(m2, radii, dep, con, row_opac, img,
                                      nnz if C == 1 else 0, C, ts, tw, th,
                                      torch.empty(nnz, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    n_isects_ref = int(state["total"][0][0])

    # fused: capacity-sized inputs and outputs, the row count on the device
    def padded(t, fill=0):
        full = torch.full((cap,) + tuple(t.shape[1:]), fill, dtype=t.dtype, device=DEV)
        full[:nnz] = t
        return full
    m2c, radc, depc, conc, opc = (padded(t) for t in (m2, radii, dep, con, row_opac))
    imgc = padded(c) if C > 1 else None
    sentinel = -7
    colors = torch.full((cap, 3), float(sentinel), device=DEV)
    tpg = torch.full((cap,), sentinel, dtype=torch.int32, device=DEV)
    starts = torch.full((cap + 1,), sentinel, dtype=torch.int64, device=DEV)
    recs = torch.full((cap, 8), float(sentinel), device=DEV)
    ws = torch.empty(query("gsplat_isect_prepare_rows_workspace_size", cap),
                     dtype=torch.uint8, device=DEV)
    n_isects = torch.empty(1, dtype=torch.int64, device=DEV)
    call("gsplat_sh_rows_fwd_isect_count", 1, C, N, coeffs.shape[-2], degree, ptr(md),
         ptr(vmd), ptr(coeffs), ptr(row_of), ptr(colors), cap, ptr(indptr[C:]),
         ptr(imgc), ptr(m2c), ptr(radc), ptr(depc), ptr(conc), ptr(opc), ts, tw, th,
         ptr(ws), ws.numel(), ptr(tpg), ptr(starts), ptr(recs), 0)
    call("gsplat_isect_row_starts", nnz, ptr(ws), ws.numel(), ptr(starts),
         ptr(n_isects), 0)
    torch.cuda.synchronize()
    assert torch.equal(colors[:nnz], colors_ref)
    assert torch.equal(tpg[:nnz], state["tiles_per_gauss"])
    assert torch.equal(starts[:nnz + 1], state["row_starts"])
    assert int(n_isects) == n_isects_ref == int(state["row_starts"][-1])
    assert torch.equal(recs[:nnz], state["records"])
    # nothing past the row count
    assert bool((tpg[nnz:] == sentinel).all()) and bool((starts[nnz + 1:] == sentinel).all())
    assert bool((recs[nnz:] == sentinel).all()) and bool((colors[nnz:] == sentinel).all())


@pytest.mark.parametrize("degree,C,stats", [(3, 1, True), (1, 3, False), (4, 2, False),
                                            (0, 1, True)])
def test_fused_colour_and_geometry_backward_matches_the_separate_passes(degree, C, stats):
    """gsplat_projection_packed_bwd_rows_sh against gsplat_sh_rows_bwd then
    gsplat_projection_packed_bwd_rows(_stats) with the SH call's v_means as
    v_means_add: every gradient (coefficients, means, quaternions, scales,
    opacities) and the densification statistics equal bit for bit."""
    from gsplat_amd.cuda import _ops
    means, quats, scales, opac, vm, K, W, H = small_scene(seed=60 + degree, N=2500, C=C)
    N = means.shape[0]
    gen = torch.Generator().manual_seed(8)
    coeffs = torch.randn(1, N, (degree + 1) ** 2 + 2, 3, generator=gen).to(DEV)
    out = _ops.projection_packed_fwd_with_row_map(
        means.to(DEV), None, quats.to(DEV), scales.to(DEV), opac.to(DEV),
        vm.to(DEV), K.to(DEV), W, H, 0.3, 0.01, 1e10, 0.0, False, 0)
    indptr, b, c, g, radii, m2, dep, con, comp, row_of = out
    nnz = m2.shape[0]
    args = (means.to(DEV)[None], None, quats.to(DEV)[None], scales.to(DEV)[None],
            vm.to(DEV)[None], K.to(DEV)[None], W, H, 0.3, 0, row_of, con, None)
    v_m2 = torch.randn(nnz, 2, generator=gen).to(DEV)
    v_dep = torch.randn(nnz, generator=gen).to(DEV)
    v_con = torch.randn(nnz, 3, generator=gen).to(DEV)
    v_col = torch.randn(nnz, 3, generator=gen).to(DEV)
    v_rop = torch.randn(nnz, generator=gen).to(DEV)

    def stats_bufs():
        if not stats:
            return None
        return (torch.randn(nnz, 2, generator=torch.Generator().manual_seed(9)).to(DEV),
                640.0, 360.0, torch.full((N,), 0.5, device=DEV),
                torch.full((N,), 2.0, device=DEV))

    v_coeffs_ref, v_means_sh = _ops.sh_rows_bwd(degree, args[0], args[4], coeffs, row_of,
                                                v_col)
    st_ref = stats_bufs()
    ref = _ops.projection_packed_bwd_rows(*args, v_m2, v_dep, v_con, None, False,
                                          v_row_opacities=v_rop, v_means_add=v_means_sh,
                                          stats=st_ref)
    st = stats_bufs()
    got = _ops.projection_packed_bwd_rows_sh(*args, v_m2, v_dep, v_con, None, degree,
                                             coeffs, v_col, v_row_opacities=v_rop,
                                             stats=st)
    torch.cuda.synchronize()
    for name, x, y in (("v_means", got[0], ref[0]), ("v_quats", got[2], ref[2]),
                       ("v_scales", got[3], ref[3]), ("v_opacities", got[4], ref[5]),
                       ("v_coeffs", got[5], v_coeffs_ref)):
        assert torch.equal(x, y), name
    if stats:
        assert torch.equal(st[3], st_ref[3]) and torch.equal(st[4], st_ref[4])
