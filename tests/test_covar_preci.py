"""quat_scale_to_covar_preci (QuatScaleToCovarCUDA.cu:37-287) on the GPU
against float64 PyTorch: the covariance R S^2 R^T, the precision as the
covariance's inverse, and the gradients of both through autograd.
Reference test: tests/test_basic.py:117-157 (its precision check is disabled
for ill-conditioned data; scales here keep the precision well conditioned)."""

import pytest
import torch

from oracle import torch_ref
from tests._util import DEV

pytestmark = pytest.mark.gpu


def _data(shape, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(shape + (4,), generator=g)
    s = torch.rand(shape + (3,), generator=g) * 0.8 + 0.2
    return q, s


def _triu(m):
    return torch.stack([m[..., 0, 0], m[..., 0, 1], m[..., 0, 2], m[..., 1, 1],
                        m[..., 1, 2], m[..., 2, 2]], dim=-1)


@pytest.mark.parametrize("triu", [False, True])
@pytest.mark.parametrize("shape", [(1000,), (3, 257), (1,)])
def test_covar_preci_fwd_bwd(triu, shape):
    from gsplat_amd.cuda._wrapper import quat_scale_to_covar_preci
    q, s = _data(shape, 1 + len(shape))
    qd = q.to(DEV).requires_grad_()
    sd = s.to(DEV).requires_grad_()
    covars, precis = quat_scale_to_covar_preci(qd, sd, triu=triu)

    q64 = q.double().requires_grad_()
    s64 = s.double().requires_grad_()
    C64 = torch_ref.quat_scale_to_covar(q64, s64)
    P64 = torch.linalg.inv(C64)
    if triu:
        C64, P64 = _triu(C64), _triu(P64)
    torch.testing.assert_close(covars.detach().cpu().double(), C64.detach(),
                               rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(precis.detach().cpu().double(), P64.detach(),
                               rtol=1e-4, atol=1e-4)

    g = torch.Generator().manual_seed(9)
    v_c = torch.randn(covars.shape, generator=g)
    v_p = torch.randn(precis.shape, generator=g) * 0.1
    (covars * v_c.to(DEV) + precis * v_p.to(DEV)).sum().backward()
    (C64 * v_c.double() + P64 * v_p.double()).sum().backward()
    for got, ref in ((qd.grad, q64.grad), (sd.grad, s64.grad)):
        err = (got.cpu().double() - ref).abs().max() / ref.abs().max()
        assert err < 1e-4, float(err)


def test_covar_only_and_no_gradient():
    from gsplat_amd.cuda import _ops
    q, s = _data((500,), 5)
    qd, sd = q.to(DEV), s.to(DEV)
    covars, precis = _ops.quat_scale_to_covar_preci_fwd(qd, sd, True, False, False)
    assert precis is None and covars.shape == (500, 3, 3)
    v_q, v_s = _ops.quat_scale_to_covar_preci_bwd(qd, sd, False, None, None)
    assert torch.equal(v_q.cpu(), torch.zeros(500, 4))
    assert torch.equal(v_s.cpu(), torch.zeros(500, 3))
