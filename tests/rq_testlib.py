"""Shared test / bench helpers: seeded synthetic inputs and oracle-built paged caches.

Input generation follows the measurement plan: seed = 1000 * config + stream
(0 K, 1 V, 2 K channel scales, 3 V channel scales, 4 sequence lengths,
5 block permutation, 6 Q).
"""
from __future__ import annotations

import math

import numpy as np
import torch

import oracle as O
from rotorquant_vllm.quantization import IsoQuantMSE, PlanarQuantMSE
from rotorquant_vllm.vllm.rq_backend import _build_rotation_matrix, _rq_total_bytes


class Params:
    """Codebooks and rotation of one RQ configuration (CPU, fp32)."""

    def __init__(self, mode="iso", k_bits=3, v_bits=3, iso_mode="fast", head_dim=128):
        if mode == "iso":
            kq = IsoQuantMSE(head_dim, k_bits, seed=42, mode=iso_mode)
            vq = kq if v_bits == k_bits else IsoQuantMSE(head_dim, v_bits, seed=42, mode=iso_mode)
        else:
            kq = PlanarQuantMSE(head_dim, k_bits, seed=42)
            vq = kq if v_bits == k_bits else PlanarQuantMSE(head_dim, v_bits, seed=42)
        self.mode, self.k_bits, self.v_bits, self.D = mode, k_bits, v_bits, head_dim
        self.kc, self.kb = kq.centroids.clone(), kq.boundaries.clone()
        self.vc, self.vb = vq.centroids.clone(), vq.boundaries.clone()
        self.R = _build_rotation_matrix(kq, head_dim, "cpu")
        RT = self.R.T.contiguous()
        self.rte, self.rto = RT[:, 0::2].contiguous(), RT[:, 1::2].contiguous()
        self.blk = 4 if mode == "iso" else 2

    def np(self):
        return dict(kc=self.kc.numpy(), vc=self.vc.numpy(), kb=self.kb.numpy(), vb=self.vb.numpy(),
                    R=self.R.numpy(), rte=self.rte.numpy(), rto=self.rto.numpy())


def gen(seed):
    return torch.Generator().manual_seed(seed)


def kv_config0(n_tokens, H, D, cfg=0, dtype=torch.float16):
    """N(0,1) * (1 + |N(0, 3)|) per (head, channel) for K and V."""
    out = []
    for stream in (0, 1):
        scale = 1 + (torch.randn(H, D, generator=gen(1000 * cfg + 2 + stream)) * 3).abs()
        out.append((torch.randn(n_tokens, H, D, generator=gen(1000 * cfg + stream)) * scale).to(dtype))
    return out


def kv_outlier_k(n_tokens, H, D, cfg, dtype=torch.float16, n_out=4, factor=10.0):
    """K N(0,1) with n_out seeded outlier channels per head scaled by `factor`; V N(0,1)."""
    k = torch.randn(n_tokens, H, D, generator=gen(1000 * cfg))
    g = gen(1000 * cfg + 2)
    for h in range(H):
        ch = torch.randperm(D, generator=g)[:n_out]
        k[:, h, ch] *= factor
    v = torch.randn(n_tokens, H, D, generator=gen(1000 * cfg + 1))
    return k.to(dtype), v.to(dtype)


def paged_layout(seq_lens, block_size, cfg, extra_blocks=8):
    """Seeded random physical block assignment.

    Returns (block_table (B, max_blocks) int32, num_blocks, slot ids per
    sequence as a list of int64 arrays).  Unused table entries are 0.
    """
    seq_lens = [int(x) for x in seq_lens]
    nblk = [(L + block_size - 1) // block_size for L in seq_lens]
    total = sum(nblk)
    num_blocks = total + extra_blocks
    perm = torch.randperm(num_blocks, generator=gen(1000 * cfg + 5)).numpy().astype(np.int32)
    max_blocks = max(max(nblk), 1)
    bt = np.zeros((len(seq_lens), max_blocks), np.int32)
    slots = []
    o = 0
    for b, L in enumerate(seq_lens):
        bt[b, :nblk[b]] = perm[o:o + nblk[b]]
        o += nblk[b]
        pos = np.arange(L)
        slots.append(bt[b, pos // block_size].astype(np.int64) * block_size + pos % block_size)
    return bt, num_blocks, slots


def build_cache_oracle(k, v, slot_ids, num_blocks, block_size, p: Params):
    """Pack (N, H, D) K/V with the CPU oracle into a fresh (NB, BS, total_bytes) cache."""
    N, H, D = k.shape
    dt = str(k.dtype).replace("torch.", "")
    kb, _ = O.to_bits(k)
    vb, _ = O.to_bits(v)
    pn = p.np()
    kp, kn = O.compress(kb, dt, pn["rte"], pn["rto"], pn["kb"], p.blk)
    vp, vn = O.compress(vb, dt, pn["rte"], pn["rto"], pn["vb"], p.blk)
    cache = np.zeros((num_blocks, block_size, _rq_total_bytes(D, H)), np.uint8)
    O.compress_store(cache, slot_ids, kp, kn, vp, vn)
    return cache


def kv_unit(n_tokens, H, D, cfg, dtype=torch.float16):
    """K, V ~ N(0, 1) (no channel scaling): attention outputs stay within a few units."""
    return (torch.randn(n_tokens, H, D, generator=gen(1000 * cfg)).to(dtype),
            torch.randn(n_tokens, H, D, generator=gen(1000 * cfg + 1)).to(dtype))


def decode_case(cfg, B, H, HQ, lens, block_size=16, p: Params | None = None, kv="config0", dtype=torch.bfloat16):
    """A decode problem: cache built by the oracle, q, block table, seq lens."""
    p = p or Params()
    bt, NB, slots = paged_layout(lens, block_size, cfg)
    total = int(sum(lens))
    if kv == "config0":
        k, v = kv_config0(total, H, p.D, cfg)
    elif kv == "unit":
        k, v = kv_unit(total, H, p.D, cfg)
    else:
        k, v = kv_outlier_k(total, H, p.D, cfg)
    cache = build_cache_oracle(k, v, np.concatenate(slots) if slots else np.zeros(0, np.int64), NB, block_size, p)
    q = torch.randn(B, HQ, p.D, generator=gen(1000 * cfg + 6)).to(dtype)
    return dict(cache=cache, bt=bt, lens=np.asarray(lens, np.int32), q=q, p=p, H=H, HQ=HQ, BS=block_size,
                sm_scale=1.0 / math.sqrt(p.D))


def ulp(x: np.ndarray, dtype: str) -> np.ndarray:
    """Spacing of the 16-bit output format at |x| (bf16: 8 significant bits, f16: 11)."""
    mant = 7 if dtype == "bfloat16" else 10
    e = np.floor(np.log2(np.maximum(np.abs(x.astype(np.float64)), 2.0 ** -14)))
    return 2.0 ** (e - mant)


def check_tolerance(got: np.ndarray, ref: np.ndarray, dtype: str, max_abs: float = 2e-2, min_cos: float = 0.999,
                    rot_block: int = 4):
    """Attention-output parity: cos >= 0.999 and |got - ref| <= max(2e-2, rounding allowance).

    The reference rounds its output twice to the 16-bit dtype: out_rot is
    rounded, rotated back through one 2x2 / 4x4 block of R, and rounded again
    (fused_paged_rq_decode.py:201-206, :308).  Two results whose unrounded
    out_rot agree to far better than 2e-2 can still round out_rot one ulp apart
    (an element of the block, carried to output d with weight |R[i][d]| <= 1,
    at most two such elements counted) and the output one more ulp apart.  So
    element d may differ by ulp(x_d) + 2 ulp(block max), x = max(|got|, |ref|).
    For bf16 values below 1 this is under 2e-2; above it the plain bound is
    unreachable for any implementation that rounds like the reference.
    Unit-scale cases additionally assert the plain max-abs <= 2e-2.
    Returns (max_abs, max_excess_over_bound, cos).
    """
    g64, r64 = got.astype(np.float64), ref.astype(np.float64)
    diff = np.abs(g64 - r64)
    x = np.maximum(np.abs(g64), np.abs(r64))
    D = x.shape[-1]
    blk = x.reshape(*x.shape[:-1], D // rot_block, rot_block).max(-1, keepdims=True)
    blk = np.broadcast_to(blk, (*x.shape[:-1], D // rot_block, rot_block)).reshape(x.shape)
    bound = np.maximum(max_abs, ulp(x, dtype) + 2 * ulp(blk, dtype))
    cs = cos_sim(got, ref)
    excess = float((diff - bound).max()) if diff.size else 0.0
    return float(diff.max()) if diff.size else 0.0, excess, cs


def cos_sim(a: np.ndarray, b: np.ndarray) -> float:
    a = a.astype(np.float64).ravel()
    b = b.astype(np.float64).ravel()
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na == 0 and nb == 0:
        return 1.0
    return float(a @ b / (na * nb))


def lens_uniform(B, lo, hi, cfg):
    return torch.randint(lo, hi + 1, (B,), generator=gen(1000 * cfg + 4)).tolist()


def lens_loguniform(B, lo, hi, cfg):
    u = torch.rand(B, generator=gen(1000 * cfg + 4), dtype=torch.float64)
    return [int(math.floor(math.exp(math.log(lo) + x * (math.log(hi) - math.log(lo))))) for x in u.tolist()]
