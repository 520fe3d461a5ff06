"""Spherical harmonics on the GPU against the PyTorch restatement
(gsplat/cuda/_torch_impl.py:686-788), forward and autograd backward; the
reference test is tests/test_basic.py:2903-2939."""

import pytest
import torch

from oracle import torch_ref
from tests._util import DEV, assert_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("degree", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("K_extra", [0, 3])
@pytest.mark.parametrize("masked", [False, True])
def test_sh_fwd_bwd(degree, K_extra, masked):
    from gsplat_amd.cuda._wrapper import spherical_harmonics
    g = torch.Generator().manual_seed(degree * 10 + K_extra)
    M = 1537
    K = (degree + 1) ** 2 + K_extra
    dirs = torch.randn(M, 3, generator=g)
    coeffs = torch.randn(M, K, 3, generator=g)
    masks = (torch.rand(M, generator=g) > 0.3) if masked else None
    v_col = torch.randn(M, 3, generator=g)

    d_gpu = dirs.to(DEV).requires_grad_()
    c_gpu = coeffs.to(DEV).requires_grad_()
    out = spherical_harmonics(degree, d_gpu, c_gpu, None if masks is None else masks.to(DEV))
    (out * v_col.to(DEV)).sum().backward()

    d_ref = dirs.double().requires_grad_()
    c_ref = coeffs.double().requires_grad_()
    ref = torch_ref.spherical_harmonics_ref(degree, d_ref, c_ref, masks)
    (ref * v_col.double()).sum().backward()

    assert_close(out, ref, rtol=1e-5, atol=1e-6, name="colors")
    assert_close(c_gpu.grad, c_ref.grad, rtol=1e-5, atol=1e-6, name="v_coeffs")
    if degree > 0:
        assert_close(d_gpu.grad, d_ref.grad, rtol=1e-4, atol=1e-5, name="v_dirs")
    else:
        assert float(d_gpu.grad.abs().max()) == 0.0


def test_sh_batch_dims_and_op_schema():
    import gsplat_amd  # noqa: F401
    dirs = torch.randn(2, 3, 100, 3, device=DEV)
    coeffs = torch.randn(2, 3, 100, 16, 3, device=DEV)
    out = torch.ops.gsplat.spherical_harmonics_fwd(3, dirs, coeffs, None)
    assert out.shape == (2, 3, 100, 3)
    ref = torch_ref.spherical_harmonics_ref(3, dirs.cpu().double(), coeffs.cpu().double())
    assert_close(out, ref, rtol=1e-5, atol=1e-6, name="colors")
