"""Densification statistics (gsplat/strategy/default.py:218-268) through the
C-ABI (gsplat_grad2d_stats) against the float64 host restatement: packed rows
with one and several cameras per Gaussian, dense rows with culled entries,
and accumulation onto existing state."""

import pytest
import torch

from oracle import torch_ref
from tests._util import DEV

pytestmark = pytest.mark.gpu


def _check(got, ref):
    # float32 scale, norm and atomic accumulation against float64
    torch.testing.assert_close(got.cpu().double(), ref, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("n_cameras", [1, 3])
def test_grad2d_stats_packed(n_cameras):
    from gsplat_amd.strategy.stats import accumulate_grad2d_stats
    g = torch.Generator().manual_seed(n_cameras)
    N = 50_000
    ids = torch.cat([torch.randperm(N, generator=g)[: N // 2] for _ in range(n_cameras)])
    grads = torch.randn(ids.numel(), 2, generator=g) * 1e-3
    prev_g = torch.rand(N, generator=g)
    prev_c = torch.randint(0, 5, (N,), generator=g).float()
    means2d = grads.to(DEV)
    means2d.absgrad = means2d
    info = {"means2d": means2d, "gaussian_ids": ids.to(DEV), "width": 1280,
            "height": 720, "n_cameras": n_cameras}
    got_g, got_c = accumulate_grad2d_stats(info, prev_g.to(DEV), prev_c.to(DEV), N,
                                           packed=True)
    ref_g, ref_c = torch_ref.grad2d_stats_ref(grads, ids, None, N, 1280, 720,
                                              n_cameras, prev_g, prev_c)
    _check(got_g, ref_g)
    assert torch.equal(got_c.cpu().double(), ref_c)


def test_grad2d_stats_dense_with_culled_rows():
    from gsplat_amd.strategy.stats import accumulate_grad2d_stats
    g = torch.Generator().manual_seed(7)
    C, N = 4, 20_001
    grads = torch.randn(C, N, 2, generator=g) * 1e-3
    radii = torch.randint(0, 3, (C, N, 2), generator=g, dtype=torch.int32)
    means2d = torch.zeros(C, N, 2, device=DEV)
    means2d.grad = grads.to(DEV)
    info = {"means2d": means2d, "radii": radii.to(DEV), "width": 640,
            "height": 480, "n_cameras": C}
    got_g, got_c = accumulate_grad2d_stats(info, None, None, N, packed=False,
                                           absgrad=False)
    ref_g, ref_c = torch_ref.grad2d_stats_ref(grads, None, radii, N, 640, 480, C)
    _check(got_g, ref_g)
    assert torch.equal(got_c.cpu().double(), ref_c)


def test_grad2d_stats_empty_rows_leave_state():
    from gsplat_amd.cuda import _ops
    grad2d = torch.ones(10, device=DEV)
    count = torch.ones(10, device=DEV)
    _ops.grad2d_stats(torch.empty(0, 2, device=DEV),
                      torch.empty(0, dtype=torch.int64, device=DEV), None, 10,
                      640.0, 360.0, grad2d, count)
    assert torch.equal(grad2d.cpu(), torch.ones(10))
    assert torch.equal(count.cpu(), torch.ones(10))


def test_grad2d_stats_reads_unaligned_views():
    # the rasterizer's absgrad output is a view into one shared zero-filled
    # buffer and may start at a 4-byte (not 8-byte) offset
    from gsplat_amd.cuda import _ops
    g = torch.Generator().manual_seed(3)
    N = 1001
    base = torch.randn(2 * N + 1, generator=g) * 1e-3
    grads = base[1:].view(N, 2)
    ids = torch.arange(N)
    grad2d = torch.zeros(N, device=DEV)
    count = torch.zeros(N, device=DEV)
    dev_base = base.to(DEV)
    _ops.grad2d_stats(dev_base[1:].view(N, 2), ids.to(DEV), None, N, 800.0, 520.0,
                      grad2d, count)
    ref_g, ref_c = torch_ref.grad2d_stats_ref(grads, ids, None, N, 1600, 1040, 1)
    _check(grad2d, ref_g)
    assert torch.equal(count.cpu().double(), ref_c)


@pytest.mark.parametrize("C,absgrad", [(1, True), (3, True), (2, False)])
def test_grad2d_stats_fused_into_projection_backward(C, absgrad):
    """fuse_grad2d_stats: the statistics accumulated by the packed projection's
    backward pass equal the separate pass over the same step's row gradients
    (and the float64 restatement), onto existing state."""
    import gsplat_amd as gs
    from gsplat_amd.strategy.stats import accumulate_grad2d_stats, fuse_grad2d_stats
    from tests._util import small_scene
    means, quats, scales, opac, vm, K, W, H = small_scene(seed=30 + C, N=20_000, C=C)
    g = torch.Generator().manual_seed(C)
    colors = torch.rand(means.shape[0], 3, generator=g)
    prev_g = torch.rand(means.shape[0], generator=g)
    prev_c = torch.randint(0, 5, (means.shape[0],), generator=g).float()
    ins = [t.to(DEV).requires_grad_() for t in (means, quats, scales, opac, colors)]
    rc, ra, meta = gs.rasterization(*ins, vm.to(DEV), K.to(DEV), W, H, absgrad=absgrad)
    grad2d, count, fused = fuse_grad2d_stats(meta, prev_g.to(DEV).clone(),
                                             prev_c.to(DEV).clone(), means.shape[0],
                                             absgrad=absgrad)
    assert fused
    target = torch.rand(rc.shape, generator=g).to(DEV)
    if not absgrad:
        meta["means2d"].retain_grad()
    (rc - target).abs().mean().backward()
    sep_g, sep_c = accumulate_grad2d_stats(meta, prev_g.to(DEV).clone(),
                                           prev_c.to(DEV).clone(), means.shape[0],
                                           packed=True, absgrad=absgrad)
    rows = meta["means2d"].absgrad if absgrad else meta["means2d"].grad
    assert float(rows.abs().sum()) > 0
    ref_g, ref_c = torch_ref.grad2d_stats_ref(rows.cpu(), meta["gaussian_ids"].cpu(), None,
                                              means.shape[0], W, H, C, prev_g, prev_c)
    assert torch.equal(count.cpu(), sep_c.cpu())
    assert torch.equal(count.cpu().double(), ref_c)
    _check(grad2d, ref_g)
    torch.testing.assert_close(grad2d, sep_g, rtol=1e-6, atol=1e-9)


def _fused_stats_step(seed=40, N=8_000):
    import gsplat_amd as gs
    from tests._util import small_scene
    means, quats, scales, opac, vm, K, W, H = small_scene(seed=seed, N=N, C=1)
    g = torch.Generator().manual_seed(seed)
    colors = torch.rand(means.shape[0], 3, generator=g)
    ins = [t.to(DEV).requires_grad_() for t in (means, quats, scales, opac, colors)]
    rc, ra, meta = gs.rasterization(*ins, vm.to(DEV), K.to(DEV), W, H, absgrad=True)
    target = torch.rand(rc.shape, generator=g).to(DEV)
    return rc, ra, meta, target, means.shape[0]


def test_fused_stats_are_counted_once_with_a_retained_graph():
    """A second backward through a retained graph adds no statistics: the
    request is consumed by the first (strategy/default.py:235-268 runs once
    per step)."""
    from gsplat_amd.strategy.stats import accumulate_grad2d_stats, fuse_grad2d_stats
    rc, ra, meta, target, N = _fused_stats_step()
    grad2d, count, fused = fuse_grad2d_stats(meta, None, None, N)
    assert fused
    loss = (rc - target).abs().mean()
    loss.backward(retain_graph=True)
    g1, c1 = grad2d.clone(), count.clone()
    loss.backward()
    assert torch.equal(count, c1) and torch.equal(grad2d, g1)
    sep_g, sep_c = accumulate_grad2d_stats(meta, None, None, N, packed=True)
    assert float(sep_c.sum()) > 0
    assert torch.equal(count, sep_c)
    torch.testing.assert_close(grad2d, sep_g, rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("backward", [True, False])
def test_step_outputs_are_freed_without_the_cyclic_collector(backward):
    """The fused-statistics slot holds means2d weakly, so dropping a step's
    outputs frees them at once (no reference cycle through the node)."""
    import gc
    import weakref
    from gsplat_amd.strategy.stats import fuse_grad2d_stats
    gc.collect()
    gc.disable()
    try:
        rc, ra, meta, target, N = _fused_stats_step(seed=41)
        grad2d, count, _ = fuse_grad2d_stats(meta, None, None, N)
        if backward:
            (rc - target).abs().mean().backward()
            assert float(count.sum()) > 0
        refs = [weakref.ref(meta["means2d"]), weakref.ref(meta["conics"]),
                weakref.ref(rc)]
        del rc, ra, meta, target
        assert all(r() is None for r in refs), [r() is None for r in refs]
    finally:
        gc.enable()
