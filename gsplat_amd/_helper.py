"""Seeded synthetic scenes for tests and benchmarks.

The reference loads a real scene for its tests (gsplat/_helper.py:48-99,
assets/test_garden.npz); the benchmark configurations here are synthetic and
fully determined by a seed.  Tensors are generated on the CPU with
``torch.Generator().manual_seed(seed)`` in a fixed order (means, scales,
quats, opacities, colors, target) so that a CPU and a GPU run see identical
bits.  Cameras follow the OpenCV convention (x right, y down, z forward;
viewmat = world -> camera).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, Optional

import torch


def look_at_viewmat(position, target=(0.0, 0.0, 0.0), up=(0.0, -1.0, 0.0)) -> torch.Tensor:
    """World->camera matrix of a camera at `position` looking at `target`."""
    p = torch.tensor(position, dtype=torch.float64)
    z = torch.tensor(target, dtype=torch.float64) - p
    z = z / z.norm()
    x = torch.linalg.cross(z, torch.tensor(up, dtype=torch.float64))
    x = x / x.norm()
    y = torch.linalg.cross(z, x)
    R = torch.stack([x, y, z], dim=0)
    vm = torch.eye(4, dtype=torch.float64)
    vm[:3, :3] = R
    vm[:3, 3] = -R @ p
    return vm.float()


def intrinsics(f: float, width: int, height: int, cx=None, cy=None) -> torch.Tensor:
    K = torch.zeros(3, 3)
    K[0, 0] = f
    K[1, 1] = f
    K[0, 2] = width / 2.0 if cx is None else cx
    K[1, 2] = height / 2.0 if cy is None else cy
    K[2, 2] = 1.0
    return K


@dataclass
class Scene:
    name: str
    means: torch.Tensor
    quats: torch.Tensor
    scales: torch.Tensor
    opacities: torch.Tensor
    colors: torch.Tensor
    viewmats: torch.Tensor
    Ks: torch.Tensor
    width: int
    height: int
    sh_degree: Optional[int]
    target: torch.Tensor
    kwargs: Dict = field(default_factory=dict)
    log_scales: Optional[torch.Tensor] = None
    opacity_logits: Optional[torch.Tensor] = None

    def to(self, device) -> "Scene":
        out = {}
        for k, v in self.__dict__.items():
            out[k] = v.to(device) if isinstance(v, torch.Tensor) else v
        return Scene(**out)


def _gaussians(g: torch.Generator, N: int, means: torch.Tensor, scale_mu: float,
               scale_sigma: float, opac_sigma: float):
    log_scales = torch.randn(N, 3, generator=g) * scale_sigma + scale_mu
    quats = torch.randn(N, 4, generator=g)
    quats = quats / quats.norm(dim=-1, keepdim=True)
    logits = torch.randn(N, generator=g) * opac_sigma
    return log_scales, quats, logits


def _sh_colors(g: torch.Generator, N: int, degree: int) -> torch.Tensor:
    K = (degree + 1) ** 2
    dc = torch.randn(N, 1, 3, generator=g) * 0.5
    rest = torch.randn(N, K - 1, 3, generator=g) * 0.05
    return torch.cat([dc, rest], dim=1)


def make_scene(config: int, seed: int = 0, n: Optional[int] = None) -> Scene:
    """BASELINE.json configs 0-4 (``n`` overrides the Gaussian count for
    scaled-down parity runs)."""
    g = torch.Generator().manual_seed(seed)
    if config == 0:
        N = n or 10_000
        means = torch.rand(N, 3, generator=g) * 2 - 1
        means[:, 2] += 3.0
        log_scales, quats, logits = _gaussians(g, N, means, -3.0, 0.5, 1.0)
        colors = torch.rand(N, 1, 3, generator=g)
        W = H = 256
        viewmats = torch.eye(4)[None]
        Ks = intrinsics(256.0, W, H, 128.0, 128.0)[None]
        target = torch.rand(1, H, W, 3, generator=g)
        return Scene("cfg0_toy", means, quats, log_scales.exp(), torch.sigmoid(logits),
                     colors, viewmats, Ks, W, H, 0, target,
                     dict(near_plane=0.01, far_plane=100.0),
                     log_scales=log_scales, opacity_logits=logits)
    if config in (1, 4):
        N = n or (1_000_000 if config == 1 else 2_000_000)
        means = torch.randn(N, 3, generator=g) * 2.0
        log_scales, quats, logits = _gaussians(g, N, means, -4.0, 0.7, 1.5)
        colors = _sh_colors(g, N, 3)
        W, H, f = (1280, 720, 1000.0) if config == 1 else (1600, 1040, 1300.0)
        vm = torch.eye(4)
        vm[2, 3] = 6.0
        viewmats = vm[None]
        Ks = intrinsics(f, W, H)[None]
        target = torch.rand(1, H, W, 3, generator=g)
        return Scene(f"cfg{config}", means, quats, log_scales.exp(), torch.sigmoid(logits),
                     colors, viewmats, Ks, W, H, 3, target, {},
                     log_scales=log_scales, opacity_logits=logits)
    if config == 2:
        N = n or 500_000
        means = torch.randn(N, 3, generator=g) * 2.0
        log_scales, quats, logits = _gaussians(g, N, means, -4.0, 0.7, 1.5)
        colors = _sh_colors(g, N, 1)
        W, H, f = 960, 540, 800.0
        vms = []
        for k in range(8):
            th = 2 * math.pi * k / 8
            vms.append(look_at_viewmat((5 * math.cos(th), -1.0, 5 * math.sin(th))))
        viewmats = torch.stack(vms)
        Ks = intrinsics(f, W, H)[None].repeat(8, 1, 1)
        target = torch.rand(8, H, W, 4, generator=g)
        return Scene("cfg2", means, quats, log_scales.exp(), torch.sigmoid(logits), colors,
                     viewmats, Ks, W, H, 1, target, dict(render_mode="RGB+ED"),
                     log_scales=log_scales, opacity_logits=logits)
    if config == 3:
        N = n or 6_000_000
        u = torch.rand(N, 3, generator=g)
        means = (u - 0.5) * torch.tensor([40.0, 10.0, 40.0])
        log_scales, quats, logits = _gaussians(g, N, means, -4.0, 1.0, 2.0)
        colors = _sh_colors(g, N, 3)
        W, H, f = 1920, 1080, 1200.0
        viewmats = torch.eye(4)[None]
        Ks = intrinsics(f, W, H)[None]
        target = torch.zeros(1, H, W, 3)
        return Scene("cfg3", means, quats, log_scales.exp(), torch.sigmoid(logits), colors,
                     viewmats, Ks, W, H, 3, target, {},
                     log_scales=log_scales, opacity_logits=logits)
    raise ValueError(f"unknown config {config}")
