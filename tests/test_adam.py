"""Fused Adam (gsplat/cuda/csrc/AdamCUDA.cu:35-69) against the float32 host
restatement: bit-exact, masked and unmasked, single- and multi-tensor."""

import numpy as np
import pytest
import torch

from oracle import exact
from tests._util import DEV

pytestmark = pytest.mark.gpu


def _tensors(shape, seed):
    g = torch.Generator().manual_seed(seed)
    p = torch.randn(shape, generator=g)
    gr = torch.randn(shape, generator=g)
    m = torch.randn(shape, generator=g) * 0.1
    v = torch.rand(shape, generator=g) * 0.1
    return p, gr, m, v


@pytest.mark.parametrize("shape", [(1000, 3), (777, 4), (1001,), (513, 45), (3, 1)])
@pytest.mark.parametrize("masked", [False, True])
def test_adam_bitexact(shape, masked):
    import gsplat_amd as gs
    p, g, m, v = _tensors(shape, 0)
    valid = (torch.rand(shape[0]) > 0.4) if masked else None
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-15
    ep, em, ev = exact.adam(p.numpy(), g.numpy(), m.numpy(), v.numpy(),
                            None if valid is None else valid.numpy(), lr, b1, b2, eps)
    pd, gd, md, vd = (t.to(DEV) for t in (p, g, m, v))
    gs.adam(pd, gd, md, vd, None if valid is None else valid.to(DEV), lr, b1, b2, eps)
    for got, want in ((pd, ep), (md, em), (vd, ev)):
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32),
                                      want.view(np.uint32))


def test_selective_adam_one_launch_matches_per_tensor():
    """The six config-4 parameter groups in one multi-tensor launch equal the
    per-tensor oracle step."""
    import gsplat_amd as gs
    N = 4099
    shapes = [(N, 3), (N, 3), (N, 4), (N,), (N, 1, 3), (N, 15, 3)]
    lrs = [1.6e-4, 5e-3, 1e-3, 5e-2, 2.5e-3, 1.25e-4]
    params = [torch.nn.Parameter(torch.randn(s).to(DEV)) for s in shapes]
    grads = [torch.randn(s) for s in shapes]
    for prm, gr in zip(params, grads):
        prm.grad = gr.to(DEV)
    init = [prm.detach().cpu().numpy().copy() for prm in params]
    opt = gs.SelectiveAdam([{"params": [prm], "lr": lr} for prm, lr in zip(params, lrs)],
                           eps=1e-15, betas=(0.9, 0.999))
    vis = torch.rand(N) > 0.5
    opt.step(vis.to(DEV))
    for prm, p0, gr, lr in zip(params, init, grads, lrs):
        z = np.zeros_like(p0)
        ep, _, _ = exact.adam(p0, gr.numpy(), z, z, vis.numpy(), lr, 0.9, 0.999, 1e-15)
        np.testing.assert_array_equal(prm.detach().cpu().numpy().view(np.uint32),
                                      ep.view(np.uint32))


def test_adam_op_registered_and_validates():
    import gsplat_amd  # noqa: F401
    p = torch.zeros(10, 3, device=DEV)
    with pytest.raises(RuntimeError, match="valid"):
        torch.ops.gsplat.adam(p, p.clone(), p.clone(), p.clone(),
                              torch.ones(5, dtype=torch.bool, device=DEV), 1e-3, 0.9, 0.999, 1e-8)
