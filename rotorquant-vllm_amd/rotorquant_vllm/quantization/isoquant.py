"""IsoQuant parameters: one seeded unit quaternion per 4-coordinate group.

Init-time part of the reference's IsoQuantMSE (src/rotorquant_vllm/quantization/isoquant.py:46-102):
the codebook and the quaternions q_L (seed) and, in 'full' mode, q_R (seed +
10000), drawn as normalised Gaussians in the reference's order.  The generator
is the CPU's unless RQ_PARAM_DEVICE=device asks for the target device's, as the
reference uses (lloyd_max.param_draw_device).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .lloyd_max import LloydMaxCodebook, param_draw_device


def make_random_unit_quaternion(shape, device="cpu", seed: int | None = None) -> torch.Tensor:
    """(..., 4) unit quaternions [w, x, y, z] (reference: isoquant.py:46-55), drawn on
    param_draw_device(device) and returned on `device`."""
    dev = torch.device(device)
    draw = param_draw_device(dev)
    gen = torch.Generator(device=draw.type)
    if seed is not None:
        gen.manual_seed(seed)
    q = torch.randn(*shape, 4, generator=gen, device=draw)
    return (q / q.norm(dim=-1, keepdim=True).clamp(min=1e-8)).to(dev)


class IsoQuantMSE(nn.Module):
    """Quaternion block-rotation quantizer parameters ('fast': q_L only, 'full': q_L and q_R)."""

    def __init__(self, d: int, bits: int, seed: int = 42, mode: str = "fast", device="cpu"):
        super().__init__()
        if mode not in ("fast", "full"):
            raise ValueError(f"mode must be 'fast' or 'full', got {mode!r}")
        self.d = d
        self.bits = bits
        self.mode = mode
        self.n_groups = (d + 3) // 4
        self.d_padded = self.n_groups * 4
        cb = LloydMaxCodebook(d, bits)
        self.register_buffer("centroids", cb.centroids.to(device))
        self.register_buffer("boundaries", cb.boundaries.to(device))
        self.register_buffer("q_L", make_random_unit_quaternion((self.n_groups,), device=device, seed=seed))
        if mode == "full":
            self.register_buffer("q_R", make_random_unit_quaternion((self.n_groups,), device=device,
                                                                    seed=seed + 10000))
