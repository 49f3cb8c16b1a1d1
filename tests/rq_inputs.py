"""Seeded synthetic inputs of the measurement plan (tests and bench.py).

seed = 1000 * config + stream, streams: 0 K, 1 V, 2 K channel scales,
3 V channel scales, 4 sequence lengths, 5 block permutation, 6 Q.

Nothing here imports the CPU oracle: bench.py builds its device inputs from
this module, and only its cpu_baseline leg and the tests use the oracle.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from rotorquant_vllm.quantization import IsoQuantMSE, PlanarQuantMSE
from rotorquant_vllm.vllm.rq_backend import _build_rotation_matrix, _rq_total_bytes  # noqa: F401


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


def kv_unit(n_tokens, H, D, cfg, dtype=torch.float16):
    """K, V ~ N(0, 1) (no channel scaling): attention outputs stay within a few units."""
    return (torch.randn(n_tokens, H, D, generator=gen(1000 * cfg)).to(dtype),
            torch.randn(n_tokens, H, D, generator=gen(1000 * cfg + 1)).to(dtype))


def lens_uniform(B, lo, hi, cfg):
    return torch.randint(lo, hi + 1, (B,), generator=gen(1000 * cfg + 4)).tolist()


def lens_loguniform(B, lo, hi, cfg):
    u = torch.rand(B, generator=gen(1000 * cfg + 4), dtype=torch.float64)
    return [int(math.floor(math.exp(math.log(lo) + x * (math.log(hi) - math.log(lo))))) for x in u.tolist()]


def gpu_decode_inputs(lens, H=8, HQ=32, D=128, BS=16, cfg=1, mode="iso", k_bits=3, v_bits=3, iso_mode="fast",
                      copies=3, kv="config0", kv_dtype="float16", dense3=False):
    """Device inputs for a decode benchmark; the cache is filled by rq_compress_store
    (dense3: in the dense 3-bit index layout).

    kv: "config0" K and V N(0,1) * (1 + |N(0,3)|) per (head, channel); "kscale"
    only K scaled that way, V N(0,1); "outlier" K N(0,1) with 4 seeded channels
    per head at 10x, V N(0,1)."""
    from rotorquant_vllm import kernels as K

    dev = torch.device("cuda")
    p = Params(mode, k_bits, v_bits, iso_mode=iso_mode, head_dim=D)
    bt, NB, slots = paged_layout(lens, BS, cfg)
    total_bytes = (128 if dense3 else 256) * H
    cache = torch.zeros(NB, BS, total_bytes, dtype=torch.uint8, device=dev)
    slot_all = torch.from_numpy(np.concatenate(slots)).to(dev)
    g = torch.Generator(device=dev).manual_seed(1000 * cfg)
    gs = torch.Generator(device=dev).manual_seed(1000 * cfg + 2)
    k_scale = 1 + (torch.randn(H, D, generator=gs, device=dev) * 3).abs()
    v_scale = 1 + (torch.randn(H, D, generator=gs, device=dev) * 3).abs()
    if kv != "config0":
        v_scale = torch.ones(H, D, device=dev)
    if kv == "outlier":
        k_scale = torch.ones(H, D, device=dev)
        go = torch.Generator().manual_seed(1000 * cfg + 2)
        for h in range(H):
            k_scale[h, torch.randperm(D, generator=go)[:4].to(dev)] = 10.0
    kdt = getattr(torch, kv_dtype)
    rte, rto, kb, vb = (t.to(dev) for t in (p.rte, p.rto, p.kb, p.vb))
    chunk = 32768
    for s in range(0, slot_all.numel(), chunk):
        n = min(chunk, slot_all.numel() - s)
        k = (torch.randn(n, H, D, generator=g, device=dev) * k_scale).to(kdt)
        v = (torch.randn(n, H, D, generator=g, device=dev) * v_scale).to(kdt)
        K.compress_store(k, v, cache, slot_all[s:s + n], rte, rto, kb, vb, rot_block=p.blk, dense3=dense3)
    caches = [cache] + [cache.clone() for _ in range(copies - 1)]
    q = torch.randn(len(lens), HQ, D, generator=torch.Generator(device=dev).manual_seed(1000 * cfg + 6),
                    device=dev).to(torch.bfloat16)
    return dict(p=p, caches=caches, bt=torch.from_numpy(bt).to(dev), lens=torch.tensor(lens, dtype=torch.int32,
                device=dev), q=q, H=H, HQ=HQ, D=D, BS=BS, lens_host=list(lens), bt_host=bt, NB=NB, dense3=dense3)


def gpu_prefill_inputs(q_lens, ctx_lens, H, HQ, cfg, mode, bits, iso_mode="fast"):
    """Device cache holding every sequence's context (new tokens included; K scaled per
    channel as in config 0, V N(0,1), bf16) and bf16 N(0,1) queries for the new tokens."""
    inp = gpu_decode_inputs(ctx_lens, H=H, HQ=HQ, cfg=cfg, mode=mode, k_bits=bits, v_bits=bits, iso_mode=iso_mode,
                            copies=1, kv="kscale", kv_dtype="bfloat16")
    dev = inp["q"].device
    T = int(sum(q_lens))
    inp["q"] = torch.randn(T, HQ, 128, generator=torch.Generator(device=dev).manual_seed(1000 * cfg + 6),
                           device=dev).to(torch.bfloat16)
    inp["cu"] = torch.from_numpy(np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)).to(dev)
    inp["q_lens"] = list(q_lens)
    return inp


def host_subcache(cache, bt_host, lens, seqs):
    """The blocks that sequences `seqs` reference, copied from the device cache to the
    host: (sub-cache (U, BS, TB) uint8, remapped block table rows, their lengths)."""
    BS = cache.shape[1]
    rows = [np.asarray(bt_host[b][:(int(lens[b]) + BS - 1) // BS]) for b in seqs]
    uniq = np.unique(np.concatenate(rows)) if rows else np.zeros(0, np.int64)
    sub = cache.index_select(0, torch.from_numpy(uniq.astype(np.int64)).to(cache.device)).cpu().numpy()
    remap = {int(v): i for i, v in enumerate(uniq)}
    width = max((len(r) for r in rows), default=1)
    bt = np.zeros((len(seqs), max(width, 1)), np.int32)
    for i, r in enumerate(rows):
        bt[i, :len(r)] = [remap[int(v)] for v in r]
    return sub, bt, np.asarray([int(lens[b]) for b in seqs], np.int32)
