"""projection_ewa_simple_{fwd,bwd} (the op behind gsplat.cuda.proj and the
has_3dgs() probe) on the GPU against the float64 restatement
(gsplat/cuda/_torch_impl.py:42-97, 169-211), gradients against its autograd."""

import numpy as np
import pytest
import torch

from oracle import torch_ref
from tests._util import DEV, assert_close, assert_grad_close

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-5


def _inputs(seed, C=2, N=700):
    g = torch.Generator().manual_seed(seed)
    # x/z up to +-1.5: beyond the 1.3x field-of-view clamp on both sides
    z = torch.rand(C, N, generator=g) * 6 + 0.5
    xy = (torch.rand(C, N, 2, generator=g) * 3 - 1.5) * z[..., None]
    means = torch.cat([xy, z[..., None]], -1)
    A = torch.randn(C, N, 3, 3, generator=g) * 0.1
    covars = A @ A.transpose(-1, -2) + 1e-3 * torch.eye(3)
    Ks = torch.tensor([[[300.0, 0, 150.0], [0, 280.0, 100.0], [0, 0, 1]],
                       [[500.0, 0, 170.0], [0, 500.0, 90.0], [0, 0, 1]]])[:C]
    return means, covars.contiguous(), Ks.contiguous()


@pytest.mark.parametrize("camera_model", ["pinhole", "ortho"])
def test_proj_matches_float64_restatement(camera_model):
    from gsplat_amd import proj
    W, H = 300, 200
    means, covars, Ks = _inputs(1)
    g = torch.Generator().manual_seed(2)
    v_m2 = torch.randn(means.shape[:-1] + (2,), generator=g)
    v_c2 = torch.randn(means.shape[:-1] + (2, 2), generator=g)

    ins = [t.to(DEV).requires_grad_() for t in (means, covars)]
    m2, c2 = proj(ins[0], ins[1], Ks.to(DEV), W, H, camera_model)
    ((m2 * v_m2.to(DEV)).sum() + (c2 * v_c2.to(DEV)).sum()).backward()

    ref = [t.double().requires_grad_() for t in (means, covars)]
    rm2, rc2 = torch_ref.proj_ref(ref[0], ref[1], Ks.double(), W, H, camera_model)
    ((rm2 * v_m2.double()).sum() + (rc2 * v_c2.double()).sum()).backward()
    r32 = [t.float().clone().requires_grad_() for t in (means, covars)]
    fm2, fc2 = torch_ref.proj_ref(r32[0], r32[1], Ks, W, H, camera_model)
    ((fm2 * v_m2).sum() + (fc2 * v_c2).sum()).backward()

    assert_close(m2.cpu(), rm2.detach(), RTOL, ATOL, "means2d")
    assert_close(c2.cpu(), rc2.detach(), RTOL, ATOL, "covars2d")
    for name, a, b, b32 in zip(("v_means", "v_covars"), ins, ref, r32):
        print(assert_grad_close(a.grad, b.grad, b32.grad, RTOL, ATOL, name))
    if camera_model == "pinhole":
        # the clamp is exercised on both sides of both axes
        u = (means[..., :2] / means[..., 2:]).numpy()
        assert (u > 0.9).any() and (u < -0.9).any()


def test_proj_schema_op_and_probe():
    """The schema op as the reference's _Proj calls it, and has_3dgs()."""
    import gsplat_amd
    means, covars, Ks = _inputs(3, C=1, N=64)
    m2, c2 = torch.ops.gsplat.projection_ewa_simple_fwd(
        means.to(DEV), covars.to(DEV), Ks.to(DEV), 300, 200, 0)
    rm2, rc2 = torch_ref.proj_ref(means.double(), covars.double(), Ks.double(), 300, 200)
    assert_close(m2.cpu(), rm2, RTOL, ATOL, "means2d")
    assert_close(c2.cpu(), rc2, RTOL, ATOL, "covars2d")
    assert gsplat_amd.has_3dgs()
    with pytest.raises(RuntimeError, match="pinhole"):
        torch.ops.gsplat.projection_ewa_simple_fwd(
            means.to(DEV), covars.to(DEV), Ks.to(DEV), 300, 200, 2)
