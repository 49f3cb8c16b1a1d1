"""GPU: the vLLM-facing RQAttentionImpl end to end.

One prefill step (three ragged prompts) and one decode step through
RQAttentionImpl.forward, as vLLM drives it (rq_backend.py:858-1036 in the
reference): new K/V are compressed into the packed cache, then attention runs
from the cache, fused (RQ_USE_FUSED_PAGED=1: rq_fused_decode / rq_int8_prefill)
or unfused (paged decompress + fp32 attention).  After each step every cache
byte must equal the oracle's store of the same K/V, and the output must match
the oracle's attention within the parity tolerance (cos >= 0.999,
|got - ref| <= max(2e-2, ulp(x) + 2 ulp(rotation-block max))).
"""
import math
import types

import numpy as np
import pytest
import torch

import oracle as O
from rq_testlib import Params, build_cache_oracle, check_tolerance, gen, kv_config0, paged_layout

pytestmark = pytest.mark.gpu

H, HQ, D, BS = 8, 32, 128, 16


def _impl(monkeypatch, fused, mode, bits):
    monkeypatch.setenv("RQ_MODE", mode)
    monkeypatch.setenv("RQ_BITS", str(bits))
    monkeypatch.setenv("RQ_ISO_MODE", "fast")
    monkeypatch.delenv("RQ_K_BITS", raising=False)
    monkeypatch.delenv("RQ_V_BITS", raising=False)
    if fused:
        monkeypatch.setenv("RQ_USE_FUSED_PAGED", "1")
    else:
        monkeypatch.delenv("RQ_USE_FUSED_PAGED", raising=False)
    from rotorquant_vllm.vllm.rq_backend import RQAttentionImpl
    impl = RQAttentionImpl(HQ, D, 1.0 / math.sqrt(D), num_kv_heads=H)
    assert impl._fused_paged_available == fused and impl._fused_prefill_available == fused
    return impl


def _metadata(n_tokens, max_query_len, slots, bt, seq_lens, q_lens):
    d = torch.device("cuda")
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    return types.SimpleNamespace(
        num_actual_tokens=n_tokens, max_query_len=max_query_len, use_cascade=False,
        slot_mapping=torch.from_numpy(np.asarray(slots, np.int64)).to(d),
        block_table=torch.from_numpy(bt).to(d),
        seq_lens=torch.from_numpy(np.asarray(seq_lens, np.int32)).to(d),
        query_start_loc=torch.from_numpy(cu).to(d), max_seq_len=int(max(seq_lens)))


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "unfused"])
@pytest.mark.parametrize("mode,bits", [("iso", 3), ("planar", 4)])
def test_backend_prefill_then_decode(monkeypatch, fused, mode, bits):
    impl = _impl(monkeypatch, fused, mode, bits)
    p = Params(mode, bits, bits)
    pn = p.np()
    dev = torch.device("cuda")
    prompts = [150, 64, 33]
    full = [L + 1 for L in prompts]                 # room for one decoded token each
    bt, NB, slots = paged_layout(full, BS, 7)
    k_all, v_all = kv_config0(sum(full), H, D, 7, dtype=torch.bfloat16)
    offs = np.concatenate([[0], np.cumsum(full)])
    kv_cache = torch.zeros(NB, BS, 256 * H, dtype=torch.uint8, device=dev)

    # ---- prefill: every prompt token, one forward call ----------------------------
    pre_idx = np.concatenate([np.arange(offs[b], offs[b] + prompts[b]) for b in range(3)])
    pre_slots = np.concatenate([slots[b][:prompts[b]] for b in range(3)])
    T = len(pre_idx)
    q = torch.randn(T, HQ, D, generator=gen(7006)).to(torch.bfloat16)
    out = torch.empty(T, HQ, D, dtype=torch.bfloat16, device=dev)
    md = _metadata(T, max(prompts), pre_slots, bt, prompts, prompts)
    impl.forward(None, q.to(dev), k_all[pre_idx].to(dev), v_all[pre_idx].to(dev), kv_cache, md, output=out)
    torch.cuda.synchronize()
    ref_cache = build_cache_oracle(k_all[pre_idx], v_all[pre_idx], pre_slots, NB, BS, p)
    got_cache = kv_cache.cpu().numpy()
    assert np.array_equal(got_cache, ref_cache), f"prefill store: {int((got_cache != ref_cache).sum())} bytes differ"
    cu = np.concatenate([[0], np.cumsum(prompts)]).astype(np.int32)
    ref = O.prefill_attention(q.float().numpy(), cu, ref_cache, bt, np.asarray(prompts, np.int32), H, D, pn["kc"],
                              pn["vc"], pn["R"], 1.0 / math.sqrt(D), "bfloat16")
    err, excess, cs = check_tolerance(out.float().cpu().numpy(), ref, "bfloat16", rot_block=p.blk)
    print(f"prefill {mode}{bits} fused={fused}: max_abs={err:.3e} excess={excess:.3e} cos={cs:.6f}")
    assert excess <= 0 and cs >= 0.999

    # ---- decode: one new token per sequence ---------------------------------------
    dec_idx = np.array([offs[b] + prompts[b] for b in range(3)])
    dec_slots = np.array([slots[b][prompts[b]] for b in range(3)])
    qd = torch.randn(3, HQ, D, generator=gen(7106)).to(torch.bfloat16)
    outd = torch.empty(3, HQ, D, dtype=torch.bfloat16, device=dev)
    md = _metadata(3, 1, dec_slots, bt, full, [1, 1, 1])
    impl.forward(None, qd.to(dev), k_all[dec_idx].to(dev), v_all[dec_idx].to(dev), kv_cache, md, output=outd)
    torch.cuda.synchronize()
    all_idx = np.concatenate([pre_idx, dec_idx])
    ref_cache = build_cache_oracle(k_all[all_idx], v_all[all_idx], np.concatenate([pre_slots, dec_slots]), NB, BS, p)
    got_cache = kv_cache.cpu().numpy()
    assert np.array_equal(got_cache, ref_cache), f"decode store: {int((got_cache != ref_cache).sum())} bytes differ"
    ref = O.decode_attention(qd.float().numpy(), ref_cache, bt, np.asarray(full, np.int32), H, D, pn["kc"], pn["vc"],
                             pn["R"], 1.0 / math.sqrt(D), "bfloat16")
    err, excess, cs = check_tolerance(outd.float().cpu().numpy(), ref, "bfloat16", rot_block=p.blk)
    print(f"decode {mode}{bits} fused={fused}: max_abs={err:.3e} excess={excess:.3e} cos={cs:.6f}")
    assert excess <= 0 and cs >= 0.999
