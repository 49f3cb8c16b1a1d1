"""GPU: the opt-in dense 3-bit index layout (RQ_INDEX_DENSE3, RQ_DENSE_3BIT=1).

* compress_store in the dense layout writes exactly the oracle's dense store
  (oracle.compress_store(dense3=True): the oracle's bit-exact indices and norms,
  re-packed by oracle.dense3_pack) -- every cache byte, padding included;
* every reader of the cache gives on a dense cache the output it gives on the
  nibble cache of the same tokens, bit for bit: the two layouts hold the same
  indices and norms and the kernels run the same arithmetic on them (paged
  decompress, fused decode with 8, 4 and 2 kv heads per workgroup, int8
  prefill, rq_paged_attention, rq_paged_prefill);
* the backend with RQ_DENSE_3BIT=1: prefill then decode through
  RQAttentionImpl.forward, cache bytes against the oracle's dense store,
  outputs against the attention oracle.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
from rq_testlib import Params, build_cache_oracle, check_tolerance, gen, kv_config0, paged_layout

pytestmark = pytest.mark.gpu

D, BS = 128, 16


def _d(x):
    return torch.from_numpy(x).to("cuda") if isinstance(x, np.ndarray) else x.to("cuda")


def _caches(cfg, lens, H, p):
    bt, NB, slots = paged_layout(lens, BS, cfg)
    k, v = kv_config0(int(sum(lens)), H, D, cfg)
    sl = np.concatenate(slots)
    return bt, build_cache_oracle(k, v, sl, NB, BS, p), build_cache_oracle(k, v, sl, NB, BS, p, dense3=True)


@pytest.mark.parametrize("mode,dt", [("iso", torch.float16), ("planar", torch.bfloat16)])
def test_compress_store_dense_bytes_equal_oracle(mode, dt):
    from rotorquant_vllm import kernels as K
    p = Params(mode, 3, 3)
    H, N = 8, 300
    k, v = kv_config0(N, H, D, 91, dtype=dt)
    NB = 24
    slots = torch.randperm(NB * BS, generator=gen(911))[:N].numpy().astype(np.int64)
    slots[::37] = -1  # skipped slots
    ref = build_cache_oracle(k, v, slots, NB, BS, p, dense3=True)
    cache = torch.full((NB, BS, ref.shape[-1]), 0xAB, dtype=torch.uint8, device="cuda")
    keep = torch.ones(NB * BS, dtype=torch.bool)
    keep[torch.from_numpy(slots[slots >= 0])] = False
    untouched = torch.full((ref.shape[-1],), 0xAB, dtype=torch.uint8).numpy()
    print(f"dense compress_store {mode} {dt}: N={N} H={H} total_bytes={ref.shape[-1]}", flush=True)
    K.compress_store(_d(k), _d(v), cache, _d(slots), _d(p.rte), _d(p.rto), _d(p.kb), _d(p.vb), dense3=True)
    torch.cuda.synchronize()
    got = cache.cpu().numpy()
    flat_got, flat_ref = got.reshape(NB * BS, -1), ref.reshape(NB * BS, -1)
    written = ~keep.numpy()
    assert np.array_equal(flat_got[written], flat_ref[written]), int((flat_got[written] != flat_ref[written]).sum())
    assert (flat_got[keep.numpy()] == untouched).all(), "bytes outside the written slots changed"


def test_paged_decompress_dense_equals_nibble():
    from rotorquant_vllm import kernels as K
    p = Params("iso", 3, 3)
    lens = [1, 40, 300, 17]
    bt, nib, den = _caches(92, lens, 8, p)
    print("dense paged decompress: lens", lens, flush=True)
    outs = []
    for cache, dense3 in ((nib, False), (den, True)):
        k, v, rbt, cnt = K.paged_decompress(_d(cache), _d(bt), _d(np.asarray(lens, np.int32)), 8, D, _d(p.kc),
                                            _d(p.vc), torch.bfloat16, dense3=dense3)
        torch.cuda.synchronize()
        n = int(cnt.item())
        outs.append((k[:n].cpu(), v[:n].cpu(), rbt.cpu()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("H,HQ", [(8, 32), (4, 28), (2, 16), (2, 32), (3, 12)])
def test_fused_decode_dense_equals_nibble(H, HQ):
    """8, 4, 2 and 3 kv heads: the decode workgroup shapes (8 / 4 / 2 heads per
    workgroup and the one with the head count taken at run time), and a GQA group of
    16 (two MFMAs per pair of head dims)."""
    from rotorquant_vllm import kernels as K
    p = Params("iso", 3, 3, iso_mode="full" if H == 4 else "fast")
    lens = [1, 17, 33, 1000, 4099, 64]
    bt, nib, den = _caches(93 + H, lens, H, p)
    q = torch.randn(len(lens), HQ, D, generator=gen(930 + H)).to(torch.bfloat16).to("cuda")
    print(f"dense fused decode: H={H} HQ={HQ} lens={lens}", flush=True)
    outs = []
    for cache, dense3 in ((nib, False), (den, True)):
        o = K.fused_paged_rq_decode(q, _d(cache), _d(bt), _d(np.asarray(lens, np.int32)), _d(p.kc), _d(p.vc),
                                    _d(p.R), H, D, BS, dense3=dense3)
        torch.cuda.synchronize()
        outs.append(o.cpu())
    print("max diff", (outs[0].float() - outs[1].float()).abs().max().item(), flush=True)
    assert torch.equal(outs[0], outs[1])
    ref = O.decode_attention(q.float().cpu().numpy(), nib, bt, np.asarray(lens, np.int32), H, D, p.kc.numpy(),
                             p.vc.numpy(), p.R.numpy(), 1 / math.sqrt(D), "bfloat16")
    _, excess, cs = check_tolerance(outs[1].float().numpy(), ref, "bfloat16", rot_block=p.blk)
    assert excess <= 0 and cs >= 0.999


def test_prefill_and_paged_attention_dense_equal_nibble():
    from rotorquant_vllm import kernels as K
    p = Params("planar", 3, 3)
    q_lens, ctx = [1, 70, 129], [300, 70, 129 + 40]
    H, HQ = 8, 32
    bt, nib, den = _caches(95, ctx, H, p)
    q = torch.randn(sum(q_lens), HQ, D, generator=gen(950)).to(torch.bfloat16).to("cuda")
    cu = _d(np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32))
    lens = _d(np.asarray(ctx, np.int32))
    print(f"dense prefill / attention: q={q_lens} ctx={ctx}", flush=True)
    pre, att, ppf = [], [], []
    for cache, dense3 in ((nib, False), (den, True)):
        c = _d(cache)
        pre.append(K.fused_paged_rq_int8_prefill(q, c, _d(bt), lens, _d(p.kc), _d(p.vc), _d(p.R), H, D, BS,
                                                 cu_seqlens_q=cu, max_q_len=max(q_lens), max_seq_len=max(ctx),
                                                 dense3=dense3).cpu())
        att.append(K.paged_attention(q, c, _d(bt), lens, cu, max(q_lens), _d(p.kc), _d(p.vc), _d(p.R), H, D, BS,
                                     dense3=dense3).cpu())
        ppf.append(K.paged_prefill(q, c, _d(bt), lens, cu, max(q_lens), _d(p.kc), _d(p.vc), _d(p.R), H, D, BS,
                                   dense3=dense3).cpu())
        torch.cuda.synchronize()
    assert torch.equal(pre[0], pre[1])
    assert torch.equal(att[0], att[1])
    assert torch.equal(ppf[0], ppf[1]) and torch.equal(ppf[0], att[0])


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "unfused"])
def test_backend_dense3_prefill_then_decode(monkeypatch, fused):
    monkeypatch.setenv("RQ_MODE", "iso")
    monkeypatch.setenv("RQ_BITS", "3")
    monkeypatch.setenv("RQ_ISO_MODE", "fast")
    monkeypatch.delenv("RQ_K_BITS", raising=False)
    monkeypatch.delenv("RQ_V_BITS", raising=False)
    monkeypatch.setenv("RQ_DENSE_3BIT", "1")
    if fused:
        monkeypatch.setenv("RQ_USE_FUSED_PAGED", "1")
    else:
        monkeypatch.delenv("RQ_USE_FUSED_PAGED", raising=False)
    from rotorquant_vllm.vllm.rq_backend import RQAttentionBackend, RQAttentionImpl
    H, HQ = 8, 32
    impl = RQAttentionImpl(HQ, D, 1.0 / math.sqrt(D), num_kv_heads=H)
    p = Params("iso", 3, 3)
    pn = p.np()
    prompts = [150, 64, 33]
    full = [L + 1 for L in prompts]
    bt, NB, slots = paged_layout(full, BS, 96)
    shape = RQAttentionBackend.get_kv_cache_shape(NB, BS, H, D)
    assert shape == (NB, BS, 128 * H)
    kv_cache = torch.zeros(shape, dtype=torch.uint8, device="cuda")
    k_all, v_all = kv_config0(sum(full), H, D, 96, dtype=torch.bfloat16)
    offs = np.concatenate([[0], np.cumsum(full)])
    pre_idx = np.concatenate([np.arange(offs[b], offs[b] + prompts[b]) for b in range(3)])
    pre_slots = np.concatenate([slots[b][:prompts[b]] for b in range(3)])
    T = len(pre_idx)
    q = torch.randn(T, HQ, D, generator=gen(9606)).to(torch.bfloat16)
    out = torch.empty(T, HQ, D, dtype=torch.bfloat16, device="cuda")
    cu = np.concatenate([[0], np.cumsum(prompts)]).astype(np.int32)

    class MD:
        pass

    md = MD()
    md.num_actual_tokens, md.max_query_len, md.use_cascade = T, max(prompts), False
    md.slot_mapping = _d(np.asarray(pre_slots, np.int64))
    md.block_table, md.seq_lens = _d(bt), _d(np.asarray(prompts, np.int32))
    md.query_start_loc, md.max_seq_len = _d(cu), max(prompts)
    print(f"backend dense3 fused={fused}: prefill {prompts}", flush=True)
    impl.forward(None, q.to("cuda"), k_all[pre_idx].to("cuda"), v_all[pre_idx].to("cuda"), kv_cache, md, output=out)
    torch.cuda.synchronize()
    ref_cache = build_cache_oracle(k_all[pre_idx], v_all[pre_idx], pre_slots, NB, BS, p, dense3=True)
    got = kv_cache.cpu().numpy()
    assert np.array_equal(got, ref_cache), f"{int((got != ref_cache).sum())} bytes differ"
    nib = O.dense3_cache_to_nibbles(ref_cache, H, D)
    kv_dtype = "bfloat16"  # fused or not: K/V rounded to the q dtype, as the reference
    ref = O.prefill_attention(q.float().numpy(), cu, nib, bt, np.asarray(prompts, np.int32), H, D, pn["kc"],
                              pn["vc"], pn["R"], 1.0 / math.sqrt(D), "bfloat16", kv_dtype=kv_dtype)
    err, excess, cs = check_tolerance(out.float().cpu().numpy(), ref, "bfloat16", rot_block=p.blk)
    print(f"prefill: max_abs={err:.3e} excess={excess:.3e} cos={cs:.6f}", flush=True)
    assert excess <= 0 and cs >= 0.999
    # one decode step
    dec_idx = np.array([offs[b] + prompts[b] for b in range(3)])
    dec_slots = np.array([slots[b][prompts[b]] for b in range(3)])
    qd = torch.randn(3, HQ, D, generator=gen(9706)).to(torch.bfloat16)
    outd = torch.empty(3, HQ, D, dtype=torch.bfloat16, device="cuda")
    md.num_actual_tokens, md.max_query_len = 3, 1
    md.slot_mapping, md.seq_lens = _d(dec_slots.astype(np.int64)), _d(np.asarray(full, np.int32))
    md.query_start_loc, md.max_seq_len = _d(np.arange(4, dtype=np.int32)), max(full)
    impl.forward(None, qd.to("cuda"), k_all[dec_idx].to("cuda"), v_all[dec_idx].to("cuda"), kv_cache, md,
                 output=outd)
    torch.cuda.synchronize()
    all_idx = np.concatenate([pre_idx, dec_idx])
    ref_cache = build_cache_oracle(k_all[all_idx], v_all[all_idx], np.concatenate([pre_slots, dec_slots]), NB, BS, p,
                                   dense3=True)
    assert np.array_equal(kv_cache.cpu().numpy(), ref_cache)
    ref = O.decode_attention(qd.float().numpy(), O.dense3_cache_to_nibbles(ref_cache, H, D), bt,
                             np.asarray(full, np.int32), H, D, pn["kc"], pn["vc"], pn["R"], 1.0 / math.sqrt(D),
                             "bfloat16", kv_dtype=kv_dtype)
    err, excess, cs = check_tolerance(outd.float().cpu().numpy(), ref, "bfloat16", rot_block=p.blk)
    print(f"decode: max_abs={err:.3e} excess={excess:.3e} cos={cs:.6f}", flush=True)
    assert excess <= 0 and cs >= 0.999
