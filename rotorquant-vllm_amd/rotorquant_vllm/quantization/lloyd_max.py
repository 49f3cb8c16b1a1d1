"""Lloyd-Max scalar codebooks for the rotated-coordinate distribution N(0, 1/d).

Same construction as the reference (src/rotorquant_vllm/quantization/lloyd_max.py:26-86):
uniform initial centroids over +-3.5 sigma, boundaries at midpoints, centroid =
E[X | X in cell] with the outer cells cut at +-10.5 sigma, stopping when no
centroid moves by 1e-10 or after 200 iterations; final boundaries are float64
midpoints cast to fp32.  The integrals use scipy's adaptive quadrature on the
same integrand expression as the reference, because the packed cache depends
on the exact fp32 boundaries: a closed-form integral reproduces every centroid
bit for bit but not the sign of the tiny middle boundary (-3.5e-17 for 3 bits,
exactly 0 for 4 bits), which decides where exact zeros land.

Unlike the reference, results are memoised per (d, bits, use_exact): every
attention layer of a model shares one solve; and the head_dim-128 codebooks come
from a table of their fp32 bits, so startup needs no solve at all.
"""
from __future__ import annotations

import functools
import math
import os

import torch
from scipy import integrate


def param_draw_device(device) -> torch.device:
    """Device whose torch generator draws the seeded rotation parameters.

    RQ_PARAM_DEVICE=cpu (the default): the CPU generator, whatever the target
    device, so the rotations -- and every cache byte -- are the same on any
    machine (they equal the reference's draws on a CPU device).
    RQ_PARAM_DEVICE=device: the target device's own generator, as the reference
    draws them (quantization/isoquant.py:46-55, planarquant.py:26-37 with vLLM's
    device); those values depend on the device's RNG implementation.
    Any other value raises ValueError."""
    mode = os.environ.get("RQ_PARAM_DEVICE", "cpu").lower()
    if mode not in ("cpu", "device"):
        raise ValueError(f"RQ_PARAM_DEVICE must be 'cpu' or 'device', got '{mode}'")
    return torch.device("cpu") if mode == "cpu" else torch.device(device)


def beta_pdf(x: float, d: int) -> float:
    """Exact density of one coordinate of a uniformly random unit vector in R^d."""
    if abs(x) >= 1.0:
        return 0.0
    coeff = math.gamma(d / 2) / (math.sqrt(math.pi) * math.gamma((d - 1) / 2))
    return coeff * (1 - x * x) ** ((d - 3) / 2)


def gaussian_approx_pdf(x: float, d: int) -> float:
    """N(0, 1/d) density (the default model of a rotated coordinate)."""
    sigma2 = 1.0 / d
    return (1.0 / math.sqrt(2 * math.pi * sigma2)) * math.exp(-x * x / (2 * sigma2))


@functools.lru_cache(maxsize=None)
def _solve(d: int, bits: int, use_exact: bool, max_iter: int, tol: float) -> tuple[tuple, tuple, int]:
    levels = 1 << bits
    if use_exact:
        def density(x):
            return beta_pdf(x, d)
    else:
        def density(x):
            return gaussian_approx_pdf(x, d)

    def first_moment(x):
        return x * density(x)

    sigma = 1.0 / math.sqrt(d)
    lo, hi = -3.5 * sigma, 3.5 * sigma
    cents = [lo + (hi - lo) * (i + 0.5) / levels for i in range(levels)]
    iters = 0
    for iters in range(1, max_iter + 1):
        mids = [(cents[i] + cents[i + 1]) / 2.0 for i in range(levels - 1)]
        edges = [lo * 3] + mids + [hi * 3]
        moved = 0.0
        nxt = []
        for i in range(levels):
            a, b = edges[i], edges[i + 1]
            mass = integrate.quad(density, a, b)[0]
            if mass > 1e-15:
                c = integrate.quad(first_moment, a, b)[0] / mass
            else:
                c = cents[i]
            moved = max(moved, abs(c - cents[i]))
            nxt.append(c)
        cents = nxt
        if moved < tol:
            break
    bounds = [(cents[i] + cents[i + 1]) / 2.0 for i in range(levels - 1)]
    return tuple(cents), tuple(bounds), iters


# fp32 bit patterns of the Gaussian-model codebooks at head_dim 128 (the case
# every supported model uses), as the solve above produces them with the
# reference's schedule (max_iter 200, tol 1e-10): startup then needs no scipy
# solve.  A CPU test re-solves both and compares bit for bit.
_FP32_TABLE = {
    (128, 3): ((0xbe42c59b, 0xbdf34608, 0xbd88da01, 0xbcb17797, 0x3cb17797, 0x3d88da01, 0x3df34608, 0x3e42c59b),
               (0xbe1e344f, 0xbdbe1005, 0xbd3537e6, 0xa4200000, 0x3d3537e6, 0x3dbe1005, 0x3e1e344f)),
    (128, 4): ((0xbe775eb8, 0xbe3b50e6, 0xbe127ff3, 0xbde37f89, 0xbdaaaa39, 0xbd6de67f, 0xbd0c91c0, 0xbc3a0bdd,
                0x3c3a0bdd, 0x3d0c91c0, 0x3d6de67f, 0x3daaaa39, 0x3de37f89, 0x3e127ff3, 0x3e3b50e6, 0x3e775eb8),
               (0xbe5957cf, 0xbe26e86d, 0xbe021fdc, 0xbdc714e1, 0xbd90cebc, 0xbd3d3c1f, 0xbcbb14b7, 0x00000000,
                0x3cbb14b7, 0x3d3d3c1f, 0x3d90cebc, 0x3dc714e1, 0x3e021fdc, 0x3e26e86d, 0x3e5957cf)),
}


def _from_bits(words) -> torch.Tensor:
    return torch.tensor(list(words), dtype=torch.int64).to(torch.int32).view(torch.float32).clone()


def solve_lloyd_max(d: int, bits: int, use_exact: bool = False, max_iter: int = 200, tol: float = 1e-10):
    """Return (centroids fp32 [2^bits], boundaries fp32 [2^bits - 1])."""
    key = (int(d), int(bits))
    if not use_exact and max_iter == 200 and tol == 1e-10 and key in _FP32_TABLE:
        c, b = _FP32_TABLE[key]
        return _from_bits(c), _from_bits(b)
    cents, bounds, _ = _solve(int(d), int(bits), bool(use_exact), int(max_iter), float(tol))
    return torch.tensor(cents, dtype=torch.float32), torch.tensor(bounds, dtype=torch.float32)


def lloyd_max_iterations(d: int, bits: int, use_exact: bool = False) -> int:
    """Number of iterations the solve ran (200 = stopped at the cap, not converged)."""
    return _solve(int(d), int(bits), bool(use_exact), 200, 1e-10)[2]


class LloydMaxCodebook:
    """Lloyd-Max codebook for dimension d and `bits` bits (reference: lloyd_max.py:107-130)."""

    def __init__(self, d: int, bits: int, use_exact: bool = False):
        self.d = d
        self.bits = bits
        self.n_levels = 2 ** bits
        self.centroids, self.boundaries = solve_lloyd_max(d, bits, use_exact)

    def quantize(self, x: torch.Tensor) -> torch.Tensor:
        """Nearest-centroid indices."""
        return (x.unsqueeze(-1) - self.centroids.to(x.device)).abs().argmin(dim=-1)

    def dequantize(self, indices: torch.Tensor) -> torch.Tensor:
        return self.centroids.to(indices.device)[indices]

    def __repr__(self) -> str:
        return f"LloydMaxCodebook(d={self.d}, bits={self.bits}, levels={self.n_levels})"
