"""SelectiveAdam: Adam without bias correction that only updates visible rows.

Same constructor and ``step(visibility)`` as the reference optimizer
(gsplat/optimizers/selective_adam.py:20-101).  The reference issues one
``adam`` launch per parameter group; here every group with a gradient is
updated by ONE launch of the multi-tensor kernel (``gsplat_adam_multi``), a
single HBM pass over all parameters.  The per-element arithmetic is the
reference's (gsplat/cuda/csrc/AdamCUDA.cu:56-68).
"""

from __future__ import annotations

from typing import Optional

import torch

from ..cuda import _ops


class SelectiveAdam(torch.optim.Adam):
    """Adam restricted to the rows selected by a visibility mask.

    Args:
        params: iterable of parameters or dicts defining parameter groups
            (one tensor per group, as in the reference).
        eps: term added to the denominator.
        betas: coefficients of the running averages.
    """

    def __init__(self, params, eps, betas):
        super().__init__(params=params, eps=eps, betas=betas)

    @torch.no_grad()
    def step(self, visibility: Optional[torch.Tensor]):
        entries = []
        key = None
        for group in self.param_groups:
            lr = group["lr"]
            eps = group["eps"]
            beta1, beta2 = group["betas"]
            assert len(group["params"]) == 1, "more than one tensor in group"
            param = group["params"][0]
            if param.grad is None:
                continue
            state = self.state[param]
            if len(state) == 0:
                state["step"] = torch.tensor(0.0, dtype=torch.float32)
                state["exp_avg"] = torch.zeros_like(
                    param, memory_format=torch.preserve_format)
                state["exp_avg_sq"] = torch.zeros_like(
                    param, memory_format=torch.preserve_format)
            grad = param.grad
            if grad.is_sparse:
                grad = grad.to_dense()
            grad = grad.contiguous()
            valid = visibility
            if valid is not None and valid.dtype != torch.bool:
                valid = valid.bool()
            entries.append((param, grad, state["exp_avg"], state["exp_avg_sq"],
                            valid, lr))
            k = (float(beta1), float(beta2), float(eps))
            if key is None:
                key = k
            elif key != k:
                # groups with different betas/eps: flush what we have
                _ops.adam_multi(entries[:-1], *key)
                entries = entries[-1:]
                key = k
        if entries:
            _ops.adam_multi(entries, *key)
