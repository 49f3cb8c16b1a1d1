"""PlanarQuant parameters: one seeded Givens angle per coordinate pair.

Init-time part of the reference's PlanarQuantMSE (src/rotorquant_vllm/quantization/planarquant.py:26-37, :80-103):
theta = U[0, 1) * 2 pi, stored as (cos theta, sin theta), from the CPU's torch
generator unless RQ_PARAM_DEVICE=device asks for the target device's, as the
reference uses (lloyd_max.param_draw_device).
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn

from .lloyd_max import LloydMaxCodebook, param_draw_device


def make_random_rotations(n_groups: int, device="cpu", seed: int | None = None) -> torch.Tensor:
    """(n_groups, 2) [cos theta, sin theta] (reference: planarquant.py:26-37), drawn on
    param_draw_device(device) and returned on `device`."""
    dev = torch.device(device)
    draw = param_draw_device(dev)
    gen = torch.Generator(device=draw.type)
    if seed is not None:
        gen.manual_seed(seed)
    theta = torch.rand(n_groups, generator=gen, device=draw) * (2 * math.pi)
    return torch.stack([theta.cos(), theta.sin()], dim=-1).to(dev)


class PlanarQuantMSE(nn.Module):
    """2x2 Givens block-rotation quantizer parameters."""

    def __init__(self, d: int, bits: int, seed: int = 42, device="cpu"):
        super().__init__()
        self.d = d
        self.bits = bits
        self.n_groups = (d + 1) // 2
        self.d_padded = self.n_groups * 2
        cb = LloydMaxCodebook(d, bits)
        self.register_buffer("centroids", cb.centroids.to(device))
        self.register_buffer("boundaries", cb.boundaries.to(device))
        self.register_buffer("rot2", make_random_rotations(self.n_groups, device=device, seed=seed))
