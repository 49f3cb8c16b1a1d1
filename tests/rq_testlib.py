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
from rotorquant_vllm.vllm.rq_backend import _rq_total_bytes
from rq_inputs import (Params, gen, gpu_decode_inputs, gpu_prefill_inputs, host_subcache,  # noqa: F401
                       kv_config0, kv_outlier_k, kv_unit, lens_loguniform, lens_uniform, paged_layout)


def build_cache_oracle(k, v, slot_ids, num_blocks, block_size, p: Params, dense3: bool = False):
    """Pack (N, H, D) K/V with the CPU oracle into a fresh (NB, BS, total_bytes) cache
    (dense3: the dense 3-bit index layout)."""
    N, H, D = k.shape
    dt = str(k.dtype).replace("torch.", "")
    kb, _ = O.to_bits(k)
    vb, _ = O.to_bits(v)
    pn = p.np()
    kp, kn = O.compress(kb, dt, pn["rte"], pn["rto"], pn["kb"], p.blk)
    vp, vn = O.compress(vb, dt, pn["rte"], pn["rto"], pn["vb"], p.blk)
    cache = np.zeros((num_blocks, block_size, _rq_total_bytes(D, H, dense3=dense3)), np.uint8)
    O.compress_store(cache, slot_ids, kp, kn, vp, vn, dense3=dense3)
    return cache


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


def identical_keys_case(cfg=45, L=333, H=2, HQ=8, p=None):
    """A one-sequence decode case whose cached keys are all the same vector (per kv head); V varies.
    Every query head then weighs all keys equally: the output is the mean of V."""
    p = p or Params("iso", 3, 3)
    bt, NB, slots = paged_layout([L], 16, cfg)
    k, v = kv_config0(L, H, 128, cfg)
    k[:] = k[0:1]
    cache = build_cache_oracle(k, v, slots[0], NB, 16, p)
    q = torch.randn(1, HQ, 128, generator=gen(1000 * cfg + 6)).to(torch.bfloat16)
    return dict(p=p, cache=cache, bt=bt, lens=np.asarray([L], np.int32), q=q, H=H, HQ=HQ, BS=16,
                sm_scale=1 / math.sqrt(128))


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

