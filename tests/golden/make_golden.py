"""Write tests/golden/golden_cpu.npz: input/output vectors of the reference's CPU path.

The reference (tpurtell/rotorquant-vllm) is not imported: this script executes
the same torch / scipy operation sequence its CPU code runs, step for step:

  codebook   : quantization/lloyd_max.py:32-86 (scipy.integrate.quad schedule)
  q_L / q_R  : quantization/isoquant.py:46-55, :97-102 (seed 42, 10042)
  rot2       : quantization/planarquant.py:26-37, :102 (seed 42)
  R          : vllm/rq_backend.py:194-264 (4x4 / 2x2 fp32 block products)
  R^T split  : vllm/rq_backend.py:475-480
  compress   : triton/isoquant_compress.py:161-190 (norm, divide, matmul,
               bucketize, clamp, pack) -- identical planar path
  decompress : triton/isoquant_decompress.py:103-133

Library rounding (torch.norm's vector order, MKL sgemm's fma order) is
whatever torch 2.10 on this container's AVX-512 CPU does; the vectors are
therefore the black-box reference that rq_oracle.c must reproduce.

Run:  python tests/golden/make_golden.py   (~10 s)
"""
from __future__ import annotations

import math
import os

import numpy as np
import torch
from scipy import integrate

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden_cpu.npz")
D = 128
H = 8


# --- lloyd_max.py:26-86, as written there -----------------------------------
def gaussian_approx_pdf(x, d):
    sigma2 = 1.0 / d
    return (1.0 / math.sqrt(2 * math.pi * sigma2)) * math.exp(-x * x / (2 * sigma2))


def solve_lloyd_max(d, bits, max_iter=200, tol=1e-10):
    n_levels = 2 ** bits
    pdf = lambda x: gaussian_approx_pdf(x, d)  # noqa: E731
    sigma = 1.0 / math.sqrt(d)
    lo, hi = -3.5 * sigma, 3.5 * sigma
    centroids = [lo + (hi - lo) * (i + 0.5) / n_levels for i in range(n_levels)]
    for _ in range(max_iter):
        boundaries = [(centroids[i] + centroids[i + 1]) / 2.0 for i in range(n_levels - 1)]
        edges = [lo * 3] + boundaries + [hi * 3]
        new_centroids = []
        for i in range(n_levels):
            a, b = edges[i], edges[i + 1]
            numerator, _ = integrate.quad(lambda x: x * pdf(x), a, b)
            denominator, _ = integrate.quad(pdf, a, b)
            new_centroids.append(numerator / denominator if denominator > 1e-15 else centroids[i])
        max_shift = max(abs(new_centroids[i] - centroids[i]) for i in range(n_levels))
        centroids = new_centroids
        if max_shift < tol:
            break
    boundaries = [(centroids[i] + centroids[i + 1]) / 2.0 for i in range(n_levels - 1)]
    return torch.tensor(centroids, dtype=torch.float32), torch.tensor(boundaries, dtype=torch.float32)


# --- isoquant.py:46-55 / planarquant.py:26-37 --------------------------------
def unit_quaternions(n, seed):
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    q = torch.randn(n, 4, generator=gen, device="cpu")
    return q / q.norm(dim=-1, keepdim=True).clamp(min=1e-8)


def rotations2(n, seed):
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    angles = torch.rand(n, generator=gen, device="cpu") * (2 * math.pi)
    return torch.stack([angles.cos(), angles.sin()], dim=-1)


# --- rq_backend.py:194-253 ---------------------------------------------------
def build_iso_R(q_L, q_R, mode):
    R = torch.eye(D, dtype=torch.float32)
    for g in range(D // 4):
        ql_w, ql_x, ql_y, ql_z = q_L[g][0], q_L[g][1], q_L[g][2], q_L[g][3]
        M_left = torch.tensor([[ql_w, -ql_x, -ql_y, -ql_z], [ql_x, ql_w, -ql_z, ql_y],
                               [ql_y, ql_z, ql_w, -ql_x], [ql_z, -ql_y, ql_x, ql_w]], dtype=torch.float32)
        if mode == "full":
            qr_w, qr_x, qr_y, qr_z = q_R[g][0], q_R[g][1], q_R[g][2], q_R[g][3]
            M_right = torch.tensor([[qr_w, qr_x, qr_y, qr_z], [-qr_x, qr_w, -qr_z, qr_y],
                                    [-qr_y, qr_z, qr_w, -qr_x], [-qr_z, -qr_y, qr_x, qr_w]], dtype=torch.float32)
        else:
            M_right = torch.tensor([[ql_w, ql_x, ql_y, ql_z], [-ql_x, ql_w, -ql_z, ql_y],
                                    [-ql_y, ql_z, ql_w, -ql_x], [-ql_z, -ql_y, ql_x, ql_w]], dtype=torch.float32)
        R[4 * g:4 * g + 4, 4 * g:4 * g + 4] = M_left @ M_right
    return R


def build_planar_R(rot2):
    R = torch.eye(D, dtype=torch.float32)
    for g in range(D // 2):
        c, s = rot2[g, 0], rot2[g, 1]
        R[2 * g:2 * g + 2, 2 * g:2 * g + 2] = torch.tensor([[c, -s], [s, c]], dtype=torch.float32)
    return R


# --- isoquant_compress.py:161-190 / isoquant_decompress.py:103-133 -----------
def compress_cpu(x, rot_T_even, rot_T_odd, boundaries):
    N, Hh, Dd = x.shape
    M = N * Hh
    flat = x.reshape(M, Dd).float()
    raw_norms = torch.norm(flat, dim=-1, keepdim=True)
    normalized = flat / (raw_norms + 1e-10)
    rotation_T = torch.empty(Dd, Dd, dtype=torch.float32)
    rotation_T[:, 0::2] = rot_T_even
    rotation_T[:, 1::2] = rot_T_odd
    rotated = normalized @ rotation_T
    indices = torch.bucketize(rotated, boundaries).clamp(0, 2 ** 4 - 1)
    idx_u8 = indices.to(torch.uint8)
    packed = (idx_u8[:, 0::2] << 4) | idx_u8[:, 1::2]
    ties = (rotated.unsqueeze(-1) == boundaries).any(-1)
    return packed.reshape(N, Hh, Dd // 2), raw_norms.reshape(N, Hh, 1), rotated, ties


def decompress_cpu(packed, norms, centroids, dtype):
    N, Hh, half = packed.shape
    M = N * Hh
    pf = packed.reshape(M, half)
    nf = norms.reshape(M).float()
    c_hi = centroids[((pf >> 4) & 0x0F).long()].float() * nf.unsqueeze(-1)
    c_lo = centroids[(pf & 0x0F).long()].float() * nf.unsqueeze(-1)
    out = torch.zeros(M, 2 * half, dtype=torch.float32)
    out[:, 0::2] = c_hi
    out[:, 1::2] = c_lo
    return out.reshape(N, Hh, 2 * half).to(dtype)


def config0_kv(n_tokens, seed_base, dtype=torch.float16):
    """benchmark config 0 values: N(0,1) * (1 + |N(0,3)|) per (head, channel)."""
    out = []
    for stream in (0, 1):
        g = torch.Generator().manual_seed(seed_base + stream)
        gs = torch.Generator().manual_seed(seed_base + 2 + stream)
        scale = 1 + (torch.randn(H, D, generator=gs) * 3).abs()
        out.append((torch.randn(n_tokens, H, D, generator=g) * scale).to(dtype))
    return out


def special_rows(dtype):
    """Edge rows: zero vector, fp16-subnormal row, huge row, one-hot, constant, alternating."""
    rows = torch.zeros(8, D)
    rows[1] = 6e-8 * torch.arange(1, D + 1) / D * 3          # subnormal in fp16
    rows[2] = torch.linspace(-6e4, 6e4, D)                     # near fp16 max
    rows[3, 17] = 1.0                                          # one-hot
    rows[4] = 0.5                                              # constant
    rows[5] = torch.tensor([(-1.0) ** i for i in range(D)])
    rows[6] = torch.linspace(-1e-3, 1e-3, D)                   # small norm: eps matters
    g = torch.Generator().manual_seed(99)
    rows[7] = torch.randn(D, generator=g) * 1e3
    return rows.to(dtype).reshape(1, 8, D)


def bits16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main():
    out = {}
    for bits in (3, 4):
        c, b = solve_lloyd_max(D, bits)
        out[f"centroids_b{bits}"] = c.numpy()
        out[f"boundaries_b{bits}"] = b.numpy()
    q_L = unit_quaternions(D // 4, 42)
    q_R = unit_quaternions(D // 4, 42 + 10000)
    rot2 = rotations2(D // 2, 42)
    out["q_L"], out["q_R"], out["rot2"] = q_L.numpy(), q_R.numpy(), rot2.numpy()
    Rs = {"iso_fast": build_iso_R(q_L, q_R, "fast"), "iso_full": build_iso_R(q_L, q_R, "full"),
          "planar": build_planar_R(rot2)}
    k16, v16 = config0_kv(24, 0)
    kb16, _ = config0_kv(8, 50, torch.bfloat16)
    inputs = {"f16": torch.cat([k16, v16, special_rows(torch.float16)], 0),
              "bf16": torch.cat([kb16, special_rows(torch.bfloat16)], 0)}
    for name, x in inputs.items():
        out[f"x_{name}"] = bits16(x)
    for mode, R in Rs.items():
        out[f"R_{mode}"] = R.numpy()
        RT = R.T.contiguous()
        rte, rto = RT[:, 0::2].contiguous(), RT[:, 1::2].contiguous()
        for bits in (3, 4):
            c = torch.from_numpy(out[f"centroids_b{bits}"])
            b = torch.from_numpy(out[f"boundaries_b{bits}"])
            for name, x in inputs.items():
                packed, norms, rotated, ties = compress_cpu(x, rte, rto, b)
                key = f"{mode}_b{bits}_{name}"
                out[f"packed_{key}"] = packed.numpy()
                out[f"norms_{key}"] = norms.numpy()
                out[f"ties_{key}"] = np.array(int(ties.sum()))
                dt = torch.float16 if name == "f16" else torch.bfloat16
                out[f"dec_{key}"] = bits16(decompress_cpu(packed, norms, c, dt))
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {os.path.getsize(OUT)} bytes, {len(out)} arrays")


if __name__ == "__main__":
    main()
