"""GPU parity at the benchmark configurations' full sizes (benchmark configs 1-4).

Each case builds its cache on the device with the library's compress kernel
(bit-exact against the oracle in test_gpu_compress.py, up to 32768 tokens),
runs the kernel on the whole configuration, copies back the blocks the checked
sequences reference and compares with the float64 oracle over those bytes.
Tolerance as in the other parity tests: cos >= 0.999 and |got - ref| <=
max(2e-2, ulp(x) + 2 ulp(rotation-block max)) (rq_testlib.check_tolerance);
each case also prints its max-abs, the number of elements above the flat
2e-2 and the worst excess in bf16 ulps of the output.

Where the oracle would take minutes, a seeded subset is checked and stated:
config 2 checks 32 of its 256 sequences, config 4's decode part the
131072-token sequence and 31 of its 127 companions, config 3 and config 4's
chunks every 32nd query row plus the last 32 of each sequence.  Config 3 and
config 4's chunks run through both prefill kernels: rq_int8_prefill (the fused
path) against the prefill oracle, rq_paged_prefill (the non-fused path's long
queries) against the non-fused oracle (K/V rounded to the q dtype).
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
from rq_testlib import (check_tolerance, gpu_decode_inputs, gpu_prefill_inputs, host_subcache, lens_loguniform,
                        lens_uniform, ulp)

pytestmark = pytest.mark.gpu


def _report(tag, got, ref, dtype, blk):
    """Assert the tolerance; print max-abs, how many elements exceed the flat 2e-2, and
    the worst difference in units of one output ulp of its rotation block's largest
    element (the allowance is ulp(x) + 2 ulp(block max), i.e. at most 3 such units)."""
    err, excess, cs = check_tolerance(got, ref, dtype, rot_block=blk)
    diff = np.abs(got.astype(np.float64) - ref)
    x = np.maximum(np.abs(got.astype(np.float64)), np.abs(ref))
    bmax = x.reshape(*x.shape[:-1], -1, blk).max(-1, keepdims=True)
    bmax = np.broadcast_to(bmax, (*x.shape[:-1], x.shape[-1] // blk, blk)).reshape(x.shape)
    over = int((diff > 2e-2).sum())
    units = float((diff / ulp(bmax, dtype)).max())
    print(f"{tag}: n={got.size} max_abs={err:.3e} above_2e-2={over} worst={units:.2f} block-ulp "
          f"excess_over_bound={excess:.3e} cos={cs:.7f}", flush=True)
    assert np.isfinite(got).all()
    assert excess <= 0 and cs >= 0.999, tag


def _decode_check(tag, inp, check_seqs):
    from rotorquant_vllm import kernels as K
    p, dev = inp["p"], inp["q"].device
    lens = inp["lens_host"]
    print(f"{tag}: B={len(lens)} sum_L={sum(lens)} checking {len(check_seqs)} sequences", flush=True)
    out = K.fused_paged_rq_decode(inp["q"], inp["caches"][0], inp["bt"], inp["lens"], p.kc.to(dev), p.vc.to(dev),
                                  p.R.to(dev), inp["H"], 128, 16, max_seq_len=max(lens))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()[check_seqs]
    sub, bt, sl = host_subcache(inp["caches"][0], inp["bt_host"], lens, check_seqs)
    pn = p.np()
    ref = O.decode_attention(inp["q"].float().cpu().numpy()[check_seqs], sub, bt, sl, inp["H"], 128, pn["kc"],
                             pn["vc"], pn["R"], 1 / math.sqrt(128), "bfloat16")
    _report(tag, got, ref, "bfloat16", p.blk)


def test_config1_full_batch():
    """Config 1: 64 sequences, L ~ U[1024, 8192], 32 q / 8 kv heads, iso fast 3-bit; all checked."""
    lens = lens_uniform(64, 1024, 8192, 1)
    inp = gpu_decode_inputs(lens, copies=1)
    _decode_check("config1 B=64", inp, list(range(64)))


def test_config2_full_batch_seeded_subset():
    """Config 2: 256 sequences, L log-uniform [2048, 32768], planar K4/V3, K outlier channels;
    the whole batch decodes in one call, a seeded 32 of the 256 are checked."""
    lens = lens_loguniform(256, 2048, 32768, 2)
    inp = gpu_decode_inputs(lens, cfg=2, mode="planar", k_bits=4, v_bits=3, copies=1, kv="outlier")
    seqs = sorted(torch.randperm(256, generator=torch.Generator().manual_seed(2007))[:32].tolist())
    _decode_check("config2 B=256 (32 checked)", inp, seqs)
    del inp
    torch.cuda.empty_cache()


def test_config4_decode_part():
    """Config 4's decode part: 1 x 131072 + 127 x U[512, 16384] tokens, 28 q / 4 kv heads
    (GQA 7), iso full 3-bit, bf16 K/V.  The 131072-token sequence (the only input that
    takes the widest prep grid and the long-context merge passes) and a seeded 31 of the
    others are checked."""
    lens = [131072] + torch.randint(512, 16384 + 1, (127,), generator=torch.Generator().manual_seed(4004)).tolist()
    inp = gpu_decode_inputs(lens, H=4, HQ=28, cfg=4, mode="iso", iso_mode="full", copies=1, kv="kscale",
                            kv_dtype="bfloat16")
    others = sorted(1 + torch.randperm(127, generator=torch.Generator().manual_seed(4008))[:31].numpy())
    _decode_check("config4 decode B=128 (long + 31 checked)", inp, [0] + [int(x) for x in others])
    del inp
    torch.cuda.empty_cache()


def _prefill_check(tag, inp, rows_of, entry="int8"):
    """entry "int8": rq_int8_prefill (the fused path) against oracle.prefill_attention;
    "paged": rq_paged_prefill (the non-fused path's long queries) against
    oracle.unfused_attention (K/V rounded to the q dtype)."""
    from rotorquant_vllm import kernels as K
    p, dev = inp["p"], inp["q"].device
    lens, q_lens = inp["lens_host"], inp["q_lens"]
    tag = f"{entry}/{tag}"
    print(f"{tag}: seqs={len(lens)} q_tokens={sum(q_lens)} ctx={lens}", flush=True)
    if entry == "int8":
        out = K.fused_paged_rq_int8_prefill(inp["q"], inp["caches"][0], inp["bt"], inp["lens"], p.kc.to(dev),
                                            p.vc.to(dev), p.R.to(dev), inp["H"], 128, 16, cu_seqlens_q=inp["cu"],
                                            max_q_len=max(q_lens), max_seq_len=max(lens))
    else:
        out = K.paged_prefill(inp["q"], inp["caches"][0], inp["bt"], inp["lens"], inp["cu"], max(q_lens),
                              p.kc.to(dev), p.vc.to(dev), p.R.to(dev), inp["H"], 128, 16, max_seq_len=max(lens))
    torch.cuda.synchronize()
    cu = inp["cu"].cpu().numpy()
    rows = np.concatenate([cu[b] + rows_of(q_lens[b]) for b in range(len(lens))])
    sub, bt, sl = host_subcache(inp["caches"][0], inp["bt_host"], lens, list(range(len(lens))))
    pn = p.np()
    oracle_fn = O.prefill_attention if entry == "int8" else O.unfused_attention
    ref = oracle_fn(inp["q"].float().cpu().numpy(), cu, sub, bt, sl, inp["H"], 128, pn["kc"], pn["vc"], pn["R"],
                    1 / math.sqrt(128), "bfloat16", rows=rows)
    _report(tag, out.float().cpu().numpy()[rows], ref[rows], "bfloat16", p.blk)


def _sampled_rows(T):
    return np.unique(np.concatenate([np.arange(0, T, 32), np.arange(max(0, T - 32), T)]))


@pytest.mark.parametrize("entry", ["int8", "paged"])
def test_config3_full_size(entry):
    """Config 3: 8 fresh sequences x 4096 tokens, causal, 32 q / 8 kv, iso fast 4-bit, one call."""
    q_lens = [4096] * 8
    inp = gpu_prefill_inputs(q_lens, q_lens, 8, 32, 3, "iso", 4)
    _prefill_check("config3 8x4096", inp, _sampled_rows, entry)
    del inp
    torch.cuda.empty_cache()


@pytest.mark.parametrize("entry", ["int8", "paged"])
def test_config4_chunks_after_prefixes(entry):
    """Config 4's prefill part: 4 chunks of 2048 tokens after seeded prefixes U{0..14336},
    28 q / 4 kv heads, iso full 3-bit, one call."""
    pre = torch.randint(0, 14336 + 1, (4,), generator=torch.Generator().manual_seed(4005)).tolist()
    q_lens = [2048] * 4
    ctx = [x + 2048 for x in pre]
    inp = gpu_prefill_inputs(q_lens, ctx, 4, 28, 4, "iso", 3, iso_mode="full")
    _prefill_check(f"config4 chunks prefixes={pre}", inp, _sampled_rows, entry)
    del inp
    torch.cuda.empty_cache()


@pytest.mark.parametrize("path", ["fused", "unfused"])
def test_config4_one_forward(monkeypatch, path):
    """Config 4 as ONE RQAttentionImpl.forward: 128 decodes (1 x 131072 + 127 x U[512, 16384]
    context) then 4 chunks of 2048 tokens after prefixes U{0..14336}, 28 q / 4 kv heads, iso
    full 3-bit, bf16 (reference anchor: the mixed batch of rq_backend.py:957-976).  fused:
    RQ_USE_FUSED_PAGED=1 (decode kernel + rq_int8_prefill); unfused: the default path
    (decode kernel + rq_paged_prefill).  The forward first stores the 8324 new tokens' K/V:
    their slots must equal the oracle's compress-store of them byte for byte.  Then the
    131072-token decode, a seeded 31 of the other decodes and every 32nd row plus the last
    32 of each chunk are checked against the oracle over the cache as the forward left it."""
    import types

    from rq_testlib import Params

    monkeypatch.setenv("RQ_MODE", "iso")
    monkeypatch.setenv("RQ_BITS", "3")
    monkeypatch.setenv("RQ_ISO_MODE", "full")
    monkeypatch.delenv("RQ_K_BITS", raising=False)
    monkeypatch.delenv("RQ_V_BITS", raising=False)
    if path == "fused":
        monkeypatch.setenv("RQ_USE_FUSED_PAGED", "1")
    else:
        monkeypatch.delenv("RQ_USE_FUSED_PAGED", raising=False)
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
    assert impl._fused_paged_available == (path == "fused")
    T = int(sum(q_lens))
    g = torch.Generator(device=dev).manual_seed(4006)
    q = torch.randn(T, 28, 128, generator=g, device=dev).to(torch.bfloat16)
    k_new = torch.randn(T, 4, 128, generator=g, device=dev).to(torch.bfloat16)
    v_new = torch.randn(T, 4, 128, generator=g, device=dev).to(torch.bfloat16)
    bt_host = inp["bt_host"]
    slots = np.concatenate([bt_host[b, np.arange(L - ql, L) // 16].astype(np.int64) * 16 + np.arange(L - ql, L) % 16
                            for b, (L, ql) in enumerate(zip(ctx, q_lens))])
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    md = types.SimpleNamespace(num_actual_tokens=T, max_query_len=2048, use_cascade=False, causal=True,
                               slot_mapping=torch.from_numpy(slots).to(dev), block_table=inp["bt"],
                               seq_lens=inp["lens"], query_start_loc=torch.from_numpy(cu).to(dev),
                               max_seq_len=max(ctx))
    md.rq_query_start_loc_cpu, md.rq_seq_lens_cpu = torch.from_numpy(cu), torch.tensor(ctx, dtype=torch.int32)
    out = torch.full_like(q, float("nan"))
    print(f"config4 one forward ({path}): {len(dec)} decodes (sum L {sum(dec)}), chunk prefixes {pre}", flush=True)
    impl.forward(None, q, k_new, v_new, inp["caches"][0], md, output=out)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all(), "every query row is written"

    # the stored new tokens, byte for byte
    p = Params("iso", 3, 3, iso_mode="full")
    pn = p.np()
    TB = inp["caches"][0].shape[2]
    ref_rows = np.zeros((T, 1, TB), np.uint8)
    kb_, _ = O.to_bits(k_new.cpu())
    vb_, _ = O.to_bits(v_new.cpu())
    kp, kn = O.compress(kb_, "bfloat16", pn["rte"], pn["rto"], pn["kb"], p.blk)
    vp, vn = O.compress(vb_, "bfloat16", pn["rte"], pn["rto"], pn["vb"], p.blk)
    O.compress_store(ref_rows, np.arange(T), kp, kn, vp, vn)
    flat = inp["caches"][0].view(-1, TB)
    got_rows = flat.index_select(0, torch.from_numpy(slots).to(dev)).cpu().numpy()
    assert np.array_equal(got_rows, ref_rows[:, 0]), f"{int((got_rows != ref_rows[:, 0]).sum())} stored bytes differ"

    # decodes: the long one and a seeded 31 of the others
    others = sorted(1 + torch.randperm(127, generator=torch.Generator().manual_seed(4008))[:31].numpy())
    dseq = [0] + [int(x) for x in others]
    sub, bt, sl = host_subcache(inp["caches"][0], bt_host, ctx, dseq)
    ref = O.decode_attention(q.float().cpu().numpy()[dseq], sub, bt, sl, 4, 128, pn["kc"], pn["vc"], pn["R"],
                             1 / math.sqrt(128), "bfloat16")
    _report(f"config4 one forward ({path}): decodes", got[dseq], ref, "bfloat16", p.blk)

    # chunks: sampled rows of each
    cseq = list(range(128, 132))
    sub, bt, sl = host_subcache(inp["caches"][0], bt_host, ctx, cseq)
    ccu = cu[128:] - cu[128]
    rows = np.concatenate([ccu[i] + _sampled_rows(2048) for i in range(4)])
    oracle_fn = O.prefill_attention if path == "fused" else O.unfused_attention
    ref = oracle_fn(q.float().cpu().numpy()[cu[128]:], ccu, sub, bt, sl, 4, 128, pn["kc"], pn["vc"], pn["R"],
                    1 / math.sqrt(128), "bfloat16", rows=rows)
    _report(f"config4 one forward ({path}): chunks", got[cu[128]:][rows], ref[rows], "bfloat16", p.blk)
    del inp
    torch.cuda.empty_cache()
