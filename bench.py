"""Benchmark: fused paged decode over the packed RotorQuant cache on one MI355X.

Workload (benchmark config 1): Llama-3-8B attention-layer shape (32 query / 8 kv
heads, head_dim 128), IsoQuant fast 3-bit K and V, 64 sequences with context
lengths uniform in [1024, 8192], block_size 16, seeded random block table; K/V
drawn as N(0,1) * (1 + |N(0,3)|) per (head, channel) and pre-compressed into
the cache by the library's own compress kernel; bf16 queries N(0,1).

A step is one fused paged decode of the whole batch (rq_fused_decode: split-KV
decode kernel + merge/back-rotation).  Three copies of the cache are rotated
between steps so the 256 MB Infinity Cache cannot serve a step's reads from
the previous one.

Algorithmic bytes per step: sum_s L_s * 136 * H_kv (each packed KV byte once)
+ sum_s ceil(L_s/16) * 4 (block table) + B * H_q * D * 2 * 2 (q in, out) + 4 B.

Prints one JSON line (rank 0).  --gpus > 1 is refused: this build targets one GPU.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "rotorquant-vllm_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 / fp16 MFMA


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


from rq_inputs import gpu_decode_inputs as build_decode_inputs  # noqa: E402  (seeded device inputs)
from rq_inputs import gpu_prefill_inputs as prefill_inputs  # noqa: E402


def config1_lens(B=64, cfg=1):
    import torch
    return torch.randint(1024, 8192 + 1, (B,), generator=torch.Generator().manual_seed(1000 * cfg + 4)).tolist()


def decode_bytes(lens, H, HQ, D, BS, dense3=False):
    """Algorithmic bytes of one decode call: each token's K/V payload once (136 B per
    head at D 128; 104 B in the dense 3-bit layout), the block-table entries, q and
    out, the lengths."""
    B = len(lens)
    per_head = (104 if dense3 else 136) * D // 128
    return (sum(lens) * per_head * H + sum((L + BS - 1) // BS for L in lens) * 4 + B * HQ * D * 2 * 2 + 4 * B)


def time_decode(inp, steps, warmup, graphs=False):
    """Time `steps` decode steps (step i reads cache copy i % copies).

    Each step is one rq_fused_decode call (prep, split-KV decode and merge
    kernels) issued through a pre-validated launcher, so the host issues a step
    in a few microseconds and the GPU does not wait for Python.  With
    graphs=True the calls are instead captured in HIP graphs and replayed (the
    replays' outputs are checked bit for bit against eager calls).  Two events
    bracket the timed steps on the launch stream (avg_ms); a second pass with an
    event after every step gives the per-step median and minimum."""
    import torch

    from rotorquant_vllm import _lib
    from rotorquant_vllm import kernels as K

    p = inp["p"]
    dev = inp["q"].device
    kc, vc, R = p.kc.to(dev), p.vc.to(dev), p.R.to(dev)
    max_len = max(inp["lens_host"])
    caches = inp["caches"]
    n = len(caches)
    need = _lib.load().rq_fused_decode_workspace_bytes(len(inp["lens_host"]), inp["HQ"], inp["D"], max_len)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    outs = [torch.empty_like(inp["q"]) for _ in range(n)]

    launchers = [K.fused_paged_rq_decode_launcher(inp["q"], caches[i], inp["bt"], inp["lens"], kc, vc, R, inp["H"],
                                                  inp["D"], inp["BS"], out=outs[i], max_seq_len=max_len, workspace=ws,
                                                  dense3=inp.get("dense3", False))
                 for i in range(n)]

    def call(i):
        launchers[i % n]()

    for i in range(n):
        call(i)
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    g_list = []
    if graphs:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(n):
                call(i)
        torch.cuda.current_stream().wait_stream(side)
        for i in range(n):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                call(i)
            g_list.append(g)

    def run(i):
        if g_list:
            g_list[i % n].replay()
        else:
            call(i)

    for i in range(warmup):
        run(i)
    torch.cuda.synchronize()
    # Timed region: the steps back to back, one event before and one after (an event
    # between steps adds a few microseconds of queue work to every step).
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        run(i)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_ms = start.elapsed_time(end)
    # Per-step spread, from a second pass with an event after every step.
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record()
    for i in range(steps):
        run(i)
        ev[i + 1].record()
    torch.cuda.synchronize()
    per = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
    # The decode kernel alone (the kernel that streams the cache): a third pass of the
    # same calls, each with events recorded at that kernel's own start and end
    # (rq_fused_decode_timed launches it with hipExtLaunchKernelGGL).
    kev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    timed = [K.fused_paged_rq_decode_launcher(inp["q"], caches[i % n], inp["bt"], inp["lens"], kc, vc, R, inp["H"],
                                              inp["D"], inp["BS"], out=outs[i % n], max_seq_len=max_len, workspace=ws,
                                              dense3=inp.get("dense3", False), kernel_events=kev[i])
             for i in range(steps)]
    torch.cuda.synchronize()
    for i in range(steps):
        timed[i]()
    torch.cuda.synchronize()
    kern = sorted(a.elapsed_time(b) for a, b in kev)
    for i in range(n):  # replays must reproduce the eager results exactly
        run(i)
    torch.cuda.synchronize()
    exact = all(torch.equal(o, e) for o, e in zip(outs, eager))
    return dict(wall_s=wall, avg_ms=total_ms / steps, median_ms=per[len(per) // 2], min_ms=per[0],
                decode_kernel_avg_ms=sum(kern) / steps, decode_kernel_median_ms=kern[len(kern) // 2],
                graphs=bool(g_list), replay_matches_eager=exact), outs[0]


def time_events(fn, steps, warmup=2, warm_ms=30.0):
    """Average ms of `fn()` over `steps` calls bracketed by events on the current stream,
    after `warmup` calls and then further calls for at least `warm_ms` of wall time (the
    per-call time of a process settles only after some tens of milliseconds of work)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < warm_ms:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def decode_config(cfg, steps=10):
    """Decode throughput on benchmark config 2 (planar K4/V3, B 256, L log-uniform [2048, 32768])
    or the decode part of config 4 (Qwen2.5-7B layout, iso full 3-bit, 1 x 131072 + 127 x U[512, 16384])."""
    import torch

    from rq_inputs import lens_loguniform
    if cfg == 2:
        lens = lens_loguniform(256, 2048, 32768, 2)
        inp = build_decode_inputs(lens, cfg=2, mode="planar", k_bits=4, v_bits=3, copies=1, kv="outlier")
        H, HQ = 8, 32
    else:
        lens = [131072] + torch.randint(512, 16384 + 1, (127,), generator=torch.Generator().manual_seed(4004)).tolist()
        inp = build_decode_inputs(lens, H=4, HQ=28, cfg=4, mode="iso", iso_mode="full", copies=1, kv="kscale",
                                  kv_dtype="bfloat16")
        H, HQ = 4, 28
    t, _ = time_decode(inp, steps, 50)
    nb = decode_bytes(lens, H, HQ, 128, 16)
    gbs = nb / (t["avg_ms"] * 1e-3) / 1e9
    out = dict(batch=len(lens), sum_ctx_tokens=int(sum(lens)), us=round(t["avg_ms"] * 1e3, 1), GBps=round(gbs, 1),
               pct_hbm_peak=round(100 * gbs / HBM_PEAK_GBS, 2), decode_tok_per_s=round(len(lens) / (t["avg_ms"] * 1e-3), 1))
    del inp
    torch.cuda.empty_cache()
    return out


def prefill_call(inp):
    from rotorquant_vllm import kernels as K
    p, dev = inp["p"], inp["q"].device
    kc, vc, R = p.kc.to(dev), p.vc.to(dev), p.R.to(dev)
    out = __import__("torch").empty_like(inp["q"])

    def fn():
        K.fused_paged_rq_int8_prefill(inp["q"], inp["caches"][0], inp["bt"], inp["lens"], kc, vc, R, inp["H"], 128,
                                      inp["BS"], out=out, cu_seqlens_q=inp["cu"], max_q_len=max(inp["q_lens"]),
                                      max_seq_len=max(inp["lens_host"]))
    return fn


def causal_macs(q_lens, ctx_lens, HQ, D=128):
    """Multiply-adds of Q K^T plus P V over the causal band (query i of a sequence sees ctx - q + i + 1 keys)."""
    n = 0
    for q, c in zip(q_lens, ctx_lens):
        pre = c - q
        n += q * pre + q * (q + 1) // 2
    return 2 * n * HQ * D


def time_prefill_cfg3(steps=5):
    """benchmark config 3: 8 x 4096 new tokens, causal, 32 q / 8 kv, iso fast 4-bit, int8 MFMA.

    Algorithmic int8 ops = 2 x (Q K^T + P V multiply-adds over the causal band);
    the kernel issues three int8 MFMAs per product (hi.hi, hi.lo, lo.hi parts),
    so issued ops are about 3x that (plus the masked part of diagonal tiles)."""
    import torch
    q_lens = [4096] * 8
    inp = prefill_inputs(q_lens, q_lens, 8, 32, 3, "iso", 4)
    fn = prefill_call(inp)
    ms = time_events(fn, steps)
    ops = 2 * causal_macs(q_lens, q_lens, 32)
    tops = ops / (ms * 1e-3) / 1e12
    out = dict(tokens=sum(q_lens), us=round(ms * 1e3, 1), algorithmic_TOPS=round(tops, 1),
               issued_int8_TOPS=round(3 * tops, 1), int8_peak_TOPS=INT8_PEAK_TOPS,
               frac_peak_algorithmic=round(tops / INT8_PEAK_TOPS, 4),
               frac_peak_issued=round(3 * tops / INT8_PEAK_TOPS, 4))
    del inp
    torch.cuda.empty_cache()
    return out


def time_mixed_cfg4(steps=5):
    """benchmark config 4's chunked-prefill part: 4 chunks of 2048 new tokens, each after a seeded
    prefix of U{0..14336} cached tokens (Qwen2.5-7B layout, iso full 3-bit)."""
    import torch
    pre = torch.randint(0, 14336 + 1, (4,), generator=torch.Generator().manual_seed(4005)).tolist()
    q_lens = [2048] * 4
    ctx = [p + 2048 for p in pre]
    inp = prefill_inputs(q_lens, ctx, 4, 28, 4, "iso", 3, iso_mode="full")
    ms = time_events(prefill_call(inp), steps)
    ops = 2 * causal_macs(q_lens, ctx, 28)
    out = dict(chunks=4, prefix_tokens=pre, us=round(ms * 1e3, 1),
               algorithmic_TOPS=round(ops / (ms * 1e-3) / 1e12, 1))
    del inp
    torch.cuda.empty_cache()
    return out


def decode_config1_dense3(steps=20):
    """Config 1's decode batch with the cache in the opt-in dense 3-bit layout
    (RQ_DENSE_3BIT: 104 payload bytes per token and head instead of 136), same
    tokens and queries as the headline line; GB/s on the dense layout's bytes."""
    import torch
    lens = config1_lens()
    inp = build_decode_inputs(lens, dense3=True)
    t, _ = time_decode(inp, steps, 100)
    nb = decode_bytes(lens, 8, 32, 128, 16, dense3=True)
    gbs = nb / (t["avg_ms"] * 1e-3) / 1e9
    out = dict(us=round(t["avg_ms"] * 1e3, 1), algorithmic_bytes=int(nb), GBps=round(gbs, 1),
               pct_hbm_peak=round(100 * gbs / HBM_PEAK_GBS, 2), decode_tok_per_s=round(len(lens) / (t["avg_ms"] * 1e-3), 1))
    del inp
    torch.cuda.empty_cache()
    return out


def decode_config1_4bit(steps=20):
    """Config 1's decode batch with 4-bit K and V (RQ_BITS=4, iso fast): the same
    nibble layout and bytes as the headline line (the bits change only the
    codebooks), with 16-entry lookups instead of 8."""
    import torch
    lens = config1_lens()
    inp = build_decode_inputs(lens, k_bits=4, v_bits=4)
    t, _ = time_decode(inp, steps, 100)
    nb = decode_bytes(lens, 8, 32, 128, 16)
    gbs = nb / (t["avg_ms"] * 1e-3) / 1e9
    out = dict(k_bits=4, v_bits=4, us=round(t["avg_ms"] * 1e3, 1), algorithmic_bytes=int(nb), GBps=round(gbs, 1),
               pct_hbm_peak=round(100 * gbs / HBM_PEAK_GBS, 2), decode_tok_per_s=round(len(lens) / (t["avg_ms"] * 1e-3), 1))
    del inp
    torch.cuda.empty_cache()
    return out


def decode_config1_tp8_slice(steps=20):
    """One GPU's share of config 1 under tensor parallelism 8: the same 64 sequences
    with 1 kv head and 4 query heads (the layout a TP-8 rank holds; attention needs
    no exchange).  GB/s on that slice's algorithmic bytes."""
    import torch
    lens = config1_lens()
    # 8 rotated cache copies (8 x 41 MB): more than the 256 MB last-level cache holds
    inp = build_decode_inputs(lens, H=1, HQ=4, copies=8)
    t, _ = time_decode(inp, steps, 100)
    nb = decode_bytes(lens, 1, 4, 128, 16)
    gbs = nb / (t["avg_ms"] * 1e-3) / 1e9
    out = dict(kv_heads=1, q_heads=4, us=round(t["avg_ms"] * 1e3, 1), algorithmic_bytes=int(nb), GBps=round(gbs, 1),
               pct_hbm_peak=round(100 * gbs / HBM_PEAK_GBS, 2), decode_tok_per_s=round(len(lens) / (t["avg_ms"] * 1e-3), 1))
    del inp
    torch.cuda.empty_cache()
    return out


def unfused_call(inp, q, cu, max_q, paged_attention=False):
    """The backend's non-fused path over a prepared cache, as it dispatches: single-token
    decodes -> one rq_fused_decode call (max_seq_len = the block table's capacity, as the
    backend launches it); other queries of at most 16 tokens -> one rq_paged_attention
    call; longer ones -> one rq_paged_prefill call (workspaces allocated here, outside the
    timed calls).  paged_attention=True: rq_paged_attention for the decodes too.  Decode
    calls rotate over the cache copies of `inp` (call i reads copy i % copies), so that
    the last-level cache does not serve a step from the one before."""
    import torch

    from rotorquant_vllm import _lib
    from rotorquant_vllm import kernels as K
    p, dev = inp["p"], q.device
    kc, vc, R = p.kc.to(dev), p.vc.to(dev), p.R.to(dev)
    out = torch.empty_like(q)
    args = (q, inp["caches"][0], inp["bt"], inp["lens"], cu, max_q, kc, vc, R, inp["H"], 128, inp["BS"])
    step = [0]
    if max_q == 1 and not paged_attention:
        cap = inp["bt"].shape[1] * inp["BS"]
        B = inp["lens"].shape[0]
        ws = torch.empty(_lib.load().rq_fused_decode_workspace_bytes(B, q.shape[1], 128, cap), dtype=torch.uint8,
                         device=dev)
        launches = [K.fused_paged_rq_decode_launcher(q, c, inp["bt"], inp["lens"], kc, vc, R, inp["H"], 128, inp["BS"],
                                                     out=out, max_seq_len=cap, workspace=ws) for c in inp["caches"]]

        def fn():
            launches[step[0] % len(launches)]()
            step[0] += 1
        return fn
    if max_q <= 16:
        def fn():
            K.paged_attention(q, inp["caches"][step[0] % len(inp["caches"])], *args[2:], out=out)
            step[0] += 1
        return fn
    B = inp["lens"].shape[0]
    mx = int(inp["lens"].max())
    ws = torch.empty(_lib.load().rq_paged_prefill_workspace_bytes(B, inp["H"], mx), dtype=torch.uint8, device=dev)

    def fn():
        K.paged_prefill(*args, out=out, max_seq_len=mx, workspace=ws)
    return fn


def time_unfused(cfg, steps=5):
    """The non-fused path (K/V rounded to bf16) on config 1's decode batch as the backend
    dispatches it (rq_fused_decode; bytes as the fused decode's roofline; also
    rq_paged_attention on the same batch) or config 3's causal prefill (rq_paged_prefill;
    algorithmic bf16 flops = 2 x the causal Q K^T + P V multiply-adds)."""
    import torch
    if cfg == 1:
        lens = config1_lens()
        inp = build_decode_inputs(lens)  # three cache copies, rotated
        B = len(lens)
        cu = torch.arange(B + 1, dtype=torch.int32, device="cuda")
        ms = time_events(unfused_call(inp, inp["q"], cu, 1), max(steps, 20))
        ms_pa = time_events(unfused_call(inp, inp["q"], cu, 1, paged_attention=True), steps)
        nb = decode_bytes(lens, 8, 32, 128, 16)
        gbs = nb / (ms * 1e-3) / 1e9
        out = dict(batch=B, us=round(ms * 1e3, 1), GBps=round(gbs, 1), pct_hbm_peak=round(100 * gbs / HBM_PEAK_GBS, 2),
                   kernel="rq_fused_decode (the backend's dispatch of single-token decodes)",
                   paged_attention_us=round(ms_pa * 1e3, 1))
    else:
        q_lens = [4096] * 8
        inp = prefill_inputs(q_lens, q_lens, 8, 32, 3, "iso", 4)
        ms = time_events(unfused_call(inp, inp["q"], inp["cu"], max(q_lens)), steps)
        flops = 2 * causal_macs(q_lens, q_lens, 32)
        tf = flops / (ms * 1e-3) / 1e12
        out = dict(tokens=sum(q_lens), us=round(ms * 1e3, 1), bf16_TFLOPS=round(tf, 1),
                   frac_bf16_peak=round(tf / BF16_PEAK_TFLOPS, 4))
    del inp
    torch.cuda.empty_cache()
    return out


def time_paged_decompress(inp, steps=10):
    """rq_paged_decompress of config 1's cache (every referenced block expanded to bf16 K and V).

    Bytes: the referenced blocks' payload read (136 * H per slot, whole blocks) plus the
    16-bit K and V written (2 * H * D * 2 per slot), block table and marks ignored."""
    import torch

    from rotorquant_vllm import kernels as K
    p, dev = inp["p"], inp["q"].device
    kc, vc = p.kc.to(dev), p.vc.to(dev)
    H, D, BS = inp["H"], inp["D"], inp["BS"]
    NB = inp["caches"][0].shape[0]
    out_k = torch.empty(NB, BS, H, D, dtype=torch.bfloat16, device=dev)
    out_v = torch.empty_like(out_k)
    from rotorquant_vllm import _lib
    ws = torch.empty(_lib.load().rq_paged_decompress_workspace_bytes(NB), dtype=torch.uint8, device=dev)

    def fn():
        K.paged_decompress(inp["caches"][0], inp["bt"], inp["lens"], H, D, kc, vc, torch.bfloat16, out_k=out_k,
                           out_v=out_v, workspace=ws)
    ms = time_events(fn, steps)
    n_blocks = sum((L + BS - 1) // BS for L in inp["lens_host"])  # blocks are distinct in the seeded layout
    nbytes = n_blocks * BS * (136 * H + 2 * H * D * 2)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return dict(blocks=n_blocks, us=round(ms * 1e3, 1), GBps=round(gbs, 1), pct_hbm_peak=round(100 * gbs / HBM_PEAK_GBS, 2))


COMPRESS_BYTES_PER_TOKEN_H8 = 5192  # 2*H*D*2 read + 136*H payload written + 8 slot id, H = 8 (pad not counted)


def time_compress(n_tokens=32768, H=8, D=128, steps=20):
    """rq_compress_store of n_tokens K+V (fp16) into random slots.

    Algorithmic bytes per token (the roofline numerator): K and V rows read
    (2*H*D*2), the payload written (136*H) and the slot id (8) = 5192 at H = 8.
    The kernel also writes each slot's 960-byte zero padding (the format requires
    it: 6152 bytes per token with it), reported beside as GBps_with_pad."""
    import torch

    from rotorquant_vllm import kernels as K
    from rq_inputs import Params

    dev = torch.device("cuda")
    p = Params("iso", 3, 3)
    BS = 16
    NB = n_tokens // BS + 8
    slots = torch.randperm(NB * BS, generator=torch.Generator().manual_seed(5))[:n_tokens].to(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    # three input sets and caches, rotated (3 x 201 MB): the last-level cache (256 MB)
    # does not serve a call's reads from the call before
    sets = []
    for _ in range(3):
        cache = torch.zeros(NB, BS, 256 * H, dtype=torch.uint8, device=dev)
        k = torch.randn(n_tokens, H, D, generator=g, device=dev).to(torch.float16)
        v = torch.randn(n_tokens, H, D, generator=g, device=dev).to(torch.float16)
        sets.append((k, v, cache, slots, p.rte.to(dev), p.rto.to(dev), p.kb.to(dev), p.vb.to(dev)))
    step = [0]

    def call():
        K.compress_store(*sets[step[0] % 3], rot_block=4)
        step[0] += 1
    ms = time_events(call, steps, warmup=3)
    alg = n_tokens * (2 * H * D * 2 + 136 * H + 8)
    gbs = alg / (ms * 1e-3) / 1e9
    return dict(tokens=n_tokens, us=round(ms * 1e3, 1), GBps=round(gbs, 1),
                GBps_with_pad=round(n_tokens * (2 * H * D * 2 + 8 + 256 * H) / (ms * 1e-3) / 1e9, 1),
                roofline={"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_token": 2 * H * D * 2 + 136 * H + 8,
                          "traffic": None})


def config0_roundtrip(budget_s=10.0):
    """benchmark config 0: 2048 tokens x 8 kv heads x 128 of fp16 K and V, N(0,1) * (1 + |N(0,3)|)
    per (head, channel), iso fast 3-bit, one sequence of 128 blocks in a pool of 256
    (seeded permutation).  GPU: rq_compress_store into the cache, rq_paged_decompress back
    to fp16.  CPU baseline (reported, on the host cores): the reference's CPU fallback op
    sequence (torch: norm, divide, matmul, bucketize, pack; then lookup x norm), repeated on
    the same sample for about budget_s seconds.  The cache bytes are compared with the C
    oracle's store, and the Lloyd-Max boundary ties (a rotated coordinate exactly equal to
    a boundary: the place where the reference's CPU and Triton paths round differently)
    are counted."""
    import numpy as np
    import torch

    import oracle as O
    from rotorquant_vllm import kernels as K
    from rq_inputs import Params, kv_config0, paged_layout

    dev = torch.device("cuda")
    H, D, BS, N = 8, 128, 16, 2048
    p = Params("iso", 3, 3)
    k, v = kv_config0(N, H, D, cfg=0)
    bt, NB, slots = paged_layout([N], BS, 0, extra_blocks=128)
    cache = torch.zeros(NB, BS, 256 * H, dtype=torch.uint8, device=dev)
    kd, vd, sd = k.to(dev), v.to(dev), torch.from_numpy(slots[0]).to(dev)
    rte, rto, kb, vb = (t.to(dev) for t in (p.rte, p.rto, p.kb, p.vb))
    comp_ms = time_events(lambda: K.compress_store(kd, vd, cache, sd, rte, rto, kb, vb, rot_block=4), 20, 3)
    btd = torch.from_numpy(bt).to(dev)
    sl = torch.tensor([N], dtype=torch.int32, device=dev)
    kc, vc = p.kc.to(dev), p.vc.to(dev)
    out_k = torch.empty(N // BS, BS, H, D, dtype=torch.float16, device=dev)
    out_v = torch.empty_like(out_k)
    dec_ms = time_events(lambda: K.paged_decompress(cache, btd, sl, H, D, kc, vc, torch.float16, out_k=out_k,
                                                    out_v=out_v), 20, 3)
    torch.cuda.synchronize()
    # --- CPU side (the checker and the measured CPU baseline) ---
    pn = p.np()
    kbits, vbits = O.to_bits(k)[0], O.to_bits(v)[0]
    kp, kn, _, k_ties = O.compress(kbits, "float16", pn["rte"], pn["rto"], pn["kb"], 4, want_ties=True)
    vp, vn, _, v_ties = O.compress(vbits, "float16", pn["rte"], pn["rto"], pn["vb"], 4, want_ties=True)
    ref = np.zeros((NB, BS, 256 * H), np.uint8)
    O.compress_store(ref, slots[0], kp, kn, vp, vn)
    exact = bool(np.array_equal(cache.cpu().numpy(), ref))
    _, _, remap, _ = K.paged_decompress(cache, btd, sl, H, D, kc, vc, torch.float16, out_k=out_k, out_v=out_v)
    logical_k = out_k[remap[0].long()].reshape(N, H, D).cpu()  # compact blocks back in sequence order
    dec_exact = bool(np.array_equal(logical_k.view(torch.int16).numpy().view(np.uint16),
                                    O.round_to(O.decompress_f32(kp, kn, pn["kc"]), "float16").astype(np.float16)
                                    .view(np.uint16)))
    torch.set_num_threads(os.cpu_count() or 1)
    rte_c, rto_c, kb_c, vb_c, kc_c, vc_c = p.rte, p.rto, p.kb, p.vb, p.kc, p.vc
    reps, t0 = 0, time.perf_counter()
    while True:
        pk, nk = O.reference_cpu_compress(k, rte_c, rto_c, kb_c)
        pv, nv = O.reference_cpu_compress(v, rte_c, rto_c, vb_c)
        O.reference_cpu_decompress(pk, nk, kc_c, torch.float16)
        O.reference_cpu_decompress(pv, nv, vc_c, torch.float16)
        reps += 1
        if time.perf_counter() - t0 > budget_s:
            break
    cpu_s = (time.perf_counter() - t0) / reps
    cpu_exact = bool(np.array_equal(pk.numpy(), kp) and np.array_equal(pv.numpy(), vp))
    rt_bytes = N * (2 * H * D * 2 + 136 * H + 8) + N * (136 * H + 2 * H * D * 2)  # compress + decompress
    return dict(tokens=N, compress_store_us=round(comp_ms * 1e3, 1), paged_decompress_us=round(dec_ms * 1e3, 1),
                roundtrip_GBps=round(rt_bytes / ((comp_ms + dec_ms) * 1e-3) / 1e9, 1),
                cache_bit_exact_vs_oracle=exact, decompress_bit_exact_vs_oracle=dec_exact,
                boundary_ties={"k": k_ties, "v": v_ties, "elements": 2 * N * H * D},
                cpu_baseline={"value": round(rt_bytes / cpu_s / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
                              "kind": "port", "us_per_roundtrip": round(cpu_s * 1e6, 1),
                              "bytes_equal_to_gpu": cpu_exact,
                              "sample": f"config 0 (2048 tokens x 8 heads, K and V) compress + decompress with the "
                                        f"reference's CPU op sequence in torch, {reps} repetitions"})


def cpu_baseline(inp, gpu_out, budget_s=15.0):
    """CPU path on a bounded sample: oracle decompress of each sequence's blocks to bf16 (K and V
    rounded to the q dtype as the reference's kernel rounds them, fused_paged_rq_decode.py:146-147,
    :190-191) + torch fp32 attention (the reference has no CPU decode path).  Its outputs, rounded
    as the reference rounds (bf16 out_rot, back-rotation, bf16), are also compared with the GPU's
    output."""
    import numpy as np
    import torch

    import oracle as O
    from rq_testlib import check_tolerance

    torch.set_num_threads(os.cpu_count() or 1)
    p = inp["p"]
    cache = inp["caches"][0].cpu().numpy()
    q = inp["q"].float().cpu()
    R = p.R.numpy()
    lens = inp["lens_host"]
    H, HQ, D = inp["H"], inp["HQ"], inp["D"]
    G = HQ // H
    done_bytes = 0
    n_seq = 0
    outs = []
    t0 = time.perf_counter()
    for b, L in enumerate(lens):
        K_, V_ = O.gather_seq(cache, inp["bt_host"][b], L, H, D, p.kc.numpy(), p.vc.numpy(), kv_dtype="bfloat16")
        Kt = torch.from_numpy(K_.astype(np.float32)).repeat_interleave(G, dim=1).transpose(0, 1)
        Vt = torch.from_numpy(V_.astype(np.float32)).repeat_interleave(G, dim=1).transpose(0, 1)
        qr = torch.from_numpy(O.rotate_q(q[b].numpy(), R, "bfloat16"))
        s = torch.einsum("hd,hld->hl", qr, Kt) / math.sqrt(D)
        o = torch.einsum("hl,hld->hd", torch.softmax(s, -1), Vt)
        outs.append(O.unrotate_out(o.numpy(), R, "bfloat16"))
        done_bytes += decode_bytes([L], H, HQ, D, inp["BS"])
        n_seq += 1
        if time.perf_counter() - t0 > budget_s:
            break
    el = time.perf_counter() - t0
    got = gpu_out.float().cpu().numpy()[:n_seq]
    ref = np.stack(outs)
    err, excess, cs = check_tolerance(got, ref, "bfloat16", rot_block=p.blk)
    return dict(value=done_bytes / el / 1e9, unit="GB/s", cores=torch.get_num_threads(), kind="port",
                sample=f"{n_seq} of {len(lens)} config-1 sequences ({sum(lens[:n_seq])} tokens): oracle C "
                       f"decompress to bf16 + torch fp32 attention, {el:.1f} s", cpu=cpu_model(),
                os_cpu_count=os.cpu_count(),
                gpu_vs_cpu={"max_abs": err, "cos": round(cs, 7), "within_tolerance": bool(excess <= 0 and cs >= 0.999),
                            "tolerance": "cos >= 0.999, |d| <= max(2e-2, ulp(x) + 2 ulp(rotation-block max))"})


def time_config4_one_forward(steps=5):
    """benchmark config 4 as ONE RQAttentionImpl.forward (RQ_USE_FUSED_PAGED=1): 128 decodes
    (1 x 131072 + 127 x U[512, 16384] context) then 4 chunks of 2048 tokens after prefixes
    U{0..14336}, Qwen2.5-7B layout (28 q / 4 kv), iso full 3-bit, bf16.  The call stores the
    132 + 8192 new tokens' K/V, runs the fused decode on the decodes and the int8 prefill on
    the chunks.  Reported: wall time per forward (HIP events), with the decode part and the
    chunk part also timed alone through the same forward."""
    import types

    import numpy as np
    import torch

    from rq_inputs import gpu_decode_inputs

    os.environ.update(RQ_MODE="iso", RQ_BITS="3", RQ_ISO_MODE="full", RQ_USE_FUSED_PAGED="1")
    for var in ("RQ_K_BITS", "RQ_V_BITS"):
        os.environ.pop(var, None)
    from rotorquant_vllm.vllm.rq_backend import RQAttentionImpl

    dec = [131072] + torch.randint(512, 16384 + 1, (127,), generator=torch.Generator().manual_seed(4004)).tolist()
    pre = torch.randint(0, 14336 + 1, (4,), generator=torch.Generator().manual_seed(4005)).tolist()
    ctx = dec + [x + 2048 for x in pre]
    q_lens = [1] * len(dec) + [2048] * 4
    inp = gpu_decode_inputs(ctx, H=4, HQ=28, cfg=4, mode="iso", iso_mode="full", copies=1, kv="kscale",
                            kv_dtype="bfloat16")
    dev = inp["q"].device
    impl = RQAttentionImpl(28, 128, 128 ** -0.5, num_kv_heads=4)
    impl._max_model_len = 131072
    T = int(sum(q_lens))
    g = torch.Generator(device=dev).manual_seed(4006)
    q = torch.randn(T, 28, 128, generator=g, device=dev).to(torch.bfloat16)
    k_new = torch.randn(T, 4, 128, generator=g, device=dev).to(torch.bfloat16)
    v_new = torch.randn(T, 4, 128, generator=g, device=dev).to(torch.bfloat16)
    bt_host = inp["bt_host"]
    slots = np.concatenate([bt_host[b, (np.arange(L - ql, L)) // 16].astype(np.int64) * 16 + np.arange(L - ql, L) % 16
                            for b, (L, ql) in enumerate(zip(ctx, q_lens))])
    cu = torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32)

    def md_of(b0, b1):
        c = cu[b0:b1 + 1] - cu[b0]
        md = types.SimpleNamespace(num_actual_tokens=int(c[-1]), max_query_len=max(q_lens[b0:b1]), use_cascade=False,
                                   slot_mapping=torch.from_numpy(slots[int(cu[b0]):int(cu[b1])]).to(dev),
                                   block_table=inp["bt"][b0:b1], seq_lens=inp["lens"][b0:b1],
                                   query_start_loc=c.to(dev), max_seq_len=max(ctx[b0:b1]))
        md.rq_query_start_loc_cpu, md.rq_seq_lens_cpu = c, torch.tensor(ctx[b0:b1], dtype=torch.int32)
        return md, int(cu[b0]), int(cu[b1])

    out = torch.empty_like(q)
    res = {}
    for name, (b0, b1) in (("whole_batch", (0, 132)), ("decode_part", (0, 128)), ("chunk_part", (128, 132))):
        md, r0, r1 = md_of(b0, b1)
        fn = lambda: impl.forward(None, q[r0:r1], k_new[r0:r1], v_new[r0:r1], inp["caches"][0], md,  # noqa: E731
                                  output=out[r0:r1])
        res[name + "_us"] = round(time_events(fn, steps, warmup=2) * 1e3, 1)
    del inp
    torch.cuda.empty_cache()
    return dict(decodes=128, decode_ctx_tokens=int(sum(dec)), chunks=4, chunk_prefixes=pre, **res)


def hbm_read_probe(gib=4, reps=10):
    """Achievable HBM read bandwidth on this device, for context next to the 8 TB/s
    peak: torch's int64 sum over a `gib` GiB device buffer (a plain streaming read;
    on MI355X it reaches 5.8-6.2 TB/s, 73-77 % of the published peak)."""
    import torch
    x = torch.ones((gib << 30) // 8, dtype=torch.int64, device="cuda")
    for _ in range(3):
        x.sum()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        x.sum()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    nbytes = x.numel() * 8
    del x
    torch.cuda.empty_cache()
    gbs = nbytes / (ms * 1e-3) / 1e9
    return dict(method=f"torch int64 sum over {gib} GiB (plain streaming read)", bytes=nbytes, us=round(ms * 1e3, 1),
                GBps=round(gbs, 1), pct_hbm_peak=round(100 * gbs / HBM_PEAK_GBS, 2))


def measured_traffic(kernel="total"):
    """HBM bytes per decode call (or of one of its kernels) measured with rocprofv3 counters
    (see the JSON for the commands)."""
    p = os.path.join(ROOT, "profiles", "decode_cfg1_traffic.json")
    try:
        with open(p) as f:
            return json.load(f)["bytes_per_call"][kernel]
    except (OSError, KeyError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    # 300 warm-up calls (~30 ms): the per-call time falls for the first ~100-300 calls
    # of a process (config 1: ~105 us after 10 calls, ~89 from 300 calls on) and is
    # flat after that (1000 calls: the same)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-compress", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the config 2/3/4 side measurements")
    ap.add_argument("--only", choices=["compress", "prefill3", "decode2", "decode4", "prefill4", "paged_decompress",
                                       "config0", "config4_forward", "unfused1", "unfused3", "decode1_dense3", "decode1_4bit",
                                       "hbm_probe", "decode1_tp8"],
                    help="run one side measurement alone and print its JSON (for profiling)")
    ap.add_argument("--graphs", action="store_true", help="replay HIP graphs of the decode call instead of direct launches")
    ap.add_argument("--calib-copy", action="store_true",
                    help="first run one 256 MiB device-to-device copy (a kernel of known traffic for counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the decode path shards by (sequence, kv head) with no exchange", file=sys.stderr)
        sys.exit(2)

    import torch
    assert torch.cuda.is_available(), "bench.py needs a ROCm GPU"
    if args.calib_copy:
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.only:
        fn = {"compress": time_compress, "prefill3": time_prefill_cfg3, "decode2": lambda: decode_config(2),
              "decode4": lambda: decode_config(4), "prefill4": time_mixed_cfg4,
              "paged_decompress": lambda: time_paged_decompress(build_decode_inputs(config1_lens(), copies=1)),
              "config0": config0_roundtrip, "config4_forward": time_config4_one_forward,
              "unfused1": lambda: time_unfused(1), "unfused3": lambda: time_unfused(3),
              "decode1_dense3": decode_config1_dense3, "decode1_4bit": decode_config1_4bit, "hbm_probe": hbm_read_probe,
              "decode1_tp8": decode_config1_tp8_slice}[args.only]
        print(json.dumps({"only": args.only, **fn()}), flush=True)
        return
    lens = config1_lens()
    inp = build_decode_inputs(lens)
    torch.cuda.synchronize()
    t, gpu_out = time_decode(inp, args.steps, args.warmup, graphs=args.graphs)
    if t["graphs"] and not t["replay_matches_eager"]:
        print("bench.py: graph replay differs from eager results; timing eager launches", file=sys.stderr)
        t, gpu_out = time_decode(inp, args.steps, args.warmup, graphs=False)
    nbytes = decode_bytes(lens, 8, 32, 128, 16)
    # Headline: the median of the per-step event times (each step bracketed by events,
    # the whole call: prep, decode and merge kernels).  Roofline: the dominant kernel,
    # decode_kernel, over its own average duration (events at its start and end).
    step_s = t["median_ms"] * 1e-3
    gbs = nbytes / step_s / 1e9
    gbs_mean = nbytes / (t["avg_ms"] * 1e-3) / 1e9
    gbs_kernel = nbytes / (t["decode_kernel_avg_ms"] * 1e-3) / 1e9
    result = {
        "metric": "fused paged decode HBM GB/s (Llama-3-8B layer, iso fast 3-bit, B=64, L~U[1024,8192])",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t["wall_s"] / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)*(1+|N(0,3)|) K/V compressed into the cache; N(0,1) bf16 q)",
        "config": {"workload": "BASELINE config 1: fused paged decode, 32 q / 8 kv heads, D 128, B 64, "
                               "L~U[1024,8192], block 16, iso fast 3-bit K/V",
                   "batch": 64, "sum_ctx_tokens": int(sum(lens)), "algorithmic_bytes_per_step": int(nbytes),
                   "cache_copies_rotated": len(inp["caches"])},
        "decode_tok_per_s": round(64 / step_s, 1),
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "step_ms": {k: (round(v, 5) if isinstance(v, float) else v) for k, v in t.items() if k != "wall_s"},
        "value_basis": "algorithmic bytes / median per-step time (HIP events around each step on the launch "
                       "stream, %d steps)" % args.steps,
        "GBps_back_to_back_mean": round(gbs_mean, 1),
        "roofline": {"bound": "hbm", "achieved": round(gbs_kernel, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs_kernel / HBM_PEAK_GBS, 4), "traffic": measured_traffic("decode_kernel"),
                     "kernel": "decode_kernel (the kernel of each rq_fused_decode call that streams the cache): "
                               "algorithmic bytes per call / its average duration, from HIP events recorded at "
                               "its own start and end (hipExtLaunchKernelGGL via rq_fused_decode_timed) over %d "
                               "calls on the launch stream; traffic = its HBM bytes per call from "
                               "profiles/decode_cfg1_traffic.json (rocprofv3 FETCH_SIZE / WRITE_SIZE, calibrated)"
                               % args.steps,
                     "kernel_us": round(t["decode_kernel_avg_ms"] * 1e3, 2),
                     "call_achieved": round(gbs_mean, 1), "call_frac": round(gbs_mean / HBM_PEAK_GBS, 4),
                     "call_traffic": measured_traffic(),
                     "call": "the whole call (decode_prep_kernel + decode_kernel + decode_merge_kernel), back-to-back "
                             "mean from two HIP events around the timed calls"},
    }
    if not args.no_compress:
        result["compress"] = time_compress()
    if not args.no_extra:
        del inp["caches"][1:]
        result["paged_decompress_config1"] = time_paged_decompress(inp)
        torch.cuda.empty_cache()
        result["prefill_config3"] = time_prefill_cfg3()
        result["decode_config2"] = decode_config(2)
        result["decode_config4"] = decode_config(4)
        result["prefill_config4_chunks"] = time_mixed_cfg4()
        result["config4_one_forward"] = time_config4_one_forward()
        result["decode_config1_dense3"] = decode_config1_dense3()
        result["decode_config1_4bit"] = decode_config1_4bit()
        result["decode_config1_tp8_slice"] = decode_config1_tp8_slice()
        result["unfused_config1_decode"] = time_unfused(1)
        result["unfused_config3_prefill"] = time_unfused(3)
        probe = hbm_read_probe()
        probe["decode_value_frac_of_probe"] = round(gbs / probe["GBps"], 4)
        result["hbm_read_probe"] = probe
    if not args.no_cpu_baseline:
        result["config0_roundtrip"] = config0_roundtrip()
        result["cpu_baseline"] = cpu_baseline(inp, gpu_out)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
