"""GPU: the vLLM-facing RQAttentionImpl end to end.

One prefill step (three ragged prompts) and one decode step through
RQAttentionImpl.forward, as vLLM drives it (rq_backend.py:858-1036 in the
reference): new K/V are compressed into the packed cache, then attention runs
from the cache, fused (RQ_USE_FUSED_PAGED=1: rq_fused_decode / rq_int8_prefill)
or unfused (rq_paged_attention for short queries, rq_paged_prefill for longer
ones; or paged decompress + fp32 attention on the device, the path kept for
other head sizes).  After each step every cache byte must equal the oracle's
store of the same K/V, and the output must match the oracle's attention within
the parity tolerance (cos >= 0.999, |got - ref| <= max(2e-2, ulp(x) +
2 ulp(rotation-block max))); the rq_paged_attention / rq_paged_prefill path
against the oracle of the reference's non-fused path (K/V decompressed to the
q dtype).
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


@pytest.mark.parametrize("path", ["fused", "unfused", "unfused_torch"])
@pytest.mark.parametrize("mode,bits", [("iso", 3), ("planar", 4)])
def test_backend_prefill_then_decode(monkeypatch, path, mode, bits):
    """fused: RQ_USE_FUSED_PAGED=1; unfused: rq_paged_attention; unfused_torch: the
    device path kept for shapes rq_paged_attention does not take, forced here."""
    fused = path == "fused"
    impl = _impl(monkeypatch, fused, mode, bits)
    if path == "unfused_torch":
        import rotorquant_vllm.vllm.rq_backend as rq_backend_module
        monkeypatch.setattr(rq_backend_module, "_paged_attention_fn", None)
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
    # both paths round K/V to the q dtype, as the reference's fused kernels
    # (fused_paged_rq_decode.py:146-147, :190-191) and its non-fused pages do
    kv_dtype = "bfloat16"
    ref = O.prefill_attention(q.float().numpy(), cu, ref_cache, bt, np.asarray(prompts, np.int32), H, D, pn["kc"],
                              pn["vc"], pn["R"], 1.0 / math.sqrt(D), "bfloat16", kv_dtype=kv_dtype)
    err, excess, cs = check_tolerance(out.float().cpu().numpy(), ref, "bfloat16", rot_block=p.blk)
    print(f"prefill {mode}{bits} {path}: max_abs={err:.3e} excess={excess:.3e} cos={cs:.6f}")
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
                             pn["R"], 1.0 / math.sqrt(D), "bfloat16", kv_dtype=kv_dtype)
    err, excess, cs = check_tolerance(outd.float().cpu().numpy(), ref, "bfloat16", rot_block=p.blk)
    print(f"decode {mode}{bits} {path}: max_abs={err:.3e} excess={excess:.3e} cos={cs:.6f}")
    assert excess <= 0 and cs >= 0.999


def _mixed_setup(monkeypatch, H, HQ, mode, bits, iso_mode, ctx, q_lens, cfg, fused=True):
    """Impl + a cache holding every sequence's first ctx - q_len tokens (oracle store);
    the last q_len tokens of each sequence arrive in the forward call."""
    monkeypatch.setenv("RQ_MODE", mode)
    monkeypatch.setenv("RQ_BITS", str(bits))
    monkeypatch.setenv("RQ_ISO_MODE", iso_mode)
    monkeypatch.delenv("RQ_K_BITS", raising=False)
    monkeypatch.delenv("RQ_V_BITS", raising=False)
    if fused:
        monkeypatch.setenv("RQ_USE_FUSED_PAGED", "1")
    else:
        monkeypatch.delenv("RQ_USE_FUSED_PAGED", raising=False)
    from rotorquant_vllm.vllm.rq_backend import RQAttentionImpl
    impl = RQAttentionImpl(HQ, D, 1.0 / math.sqrt(D), num_kv_heads=H)
    p = Params(mode, bits, bits, iso_mode=iso_mode)
    bt, NB, slots = paged_layout(ctx, BS, cfg)
    k_all, v_all = kv_config0(sum(ctx), H, D, cfg, dtype=torch.bfloat16)
    offs = np.concatenate([[0], np.cumsum(ctx)])
    old_idx = np.concatenate([np.arange(offs[b], offs[b + 1] - q_lens[b]) for b in range(len(ctx))])
    new_idx = np.concatenate([np.arange(offs[b + 1] - q_lens[b], offs[b + 1]) for b in range(len(ctx))])
    old_slots = np.concatenate([slots[b][:ctx[b] - q_lens[b]] for b in range(len(ctx))])
    new_slots = np.concatenate([slots[b][ctx[b] - q_lens[b]:] for b in range(len(ctx))])
    cache0 = build_cache_oracle(k_all[old_idx], v_all[old_idx], old_slots, NB, BS, p)
    full_cache = build_cache_oracle(k_all, v_all, np.concatenate(slots), NB, BS, p)
    T = int(sum(q_lens))
    q = torch.randn(T, HQ, D, generator=gen(1000 * cfg + 6)).to(torch.bfloat16)
    md = _metadata(T, max(q_lens), new_slots, bt, ctx, q_lens)
    md.rq_query_start_loc_cpu = md.query_start_loc.cpu()
    md.rq_seq_lens_cpu = md.seq_lens.cpu()
    return impl, p, dict(bt=bt, NB=NB, k_new=k_all[new_idx], v_new=v_all[new_idx], cache0=cache0,
                         full_cache=full_cache, q=q, md=md)


def test_backend_mixed_batch_one_forward(monkeypatch):
    """vLLM's chunked-prefill batch shape in ONE forward: five decodes with long contexts
    first, then two prefill chunks (one after a 600-token prefix, one fresh), at the
    Qwen2.5-7B head layout (28 q / 4 kv, iso full 3-bit).  The decodes go to the fused
    decode and the chunks to the int8 prefill; the cache bytes equal the oracle's store
    and every output row meets the attention tolerance against the oracle.  The prefill
    workspace is the one sized at init (no growth)."""
    from rotorquant_vllm import kernels as K
    ctx = [9000, 3000, 1500, 700, 5, 800, 64]
    q_lens = [1, 1, 1, 1, 1, 200, 64]
    impl, p, c = _mixed_setup(monkeypatch, 4, 28, "iso", 3, "full", ctx, q_lens, 71)
    dev = torch.device("cuda")
    kv_cache = torch.from_numpy(c["cache0"]).to(dev)
    out = torch.empty(c["q"].shape, dtype=torch.bfloat16, device=dev)
    n_retired = len(K._ws_retired)
    impl.forward(None, c["q"].to(dev), c["k_new"].to(dev), c["v_new"].to(dev), kv_cache, c["md"], output=out)
    torch.cuda.synchronize()
    assert len(K._ws_retired) == n_retired, "the forward grew a workspace"
    got_cache = kv_cache.cpu().numpy()
    assert np.array_equal(got_cache, c["full_cache"]), f"{int((got_cache != c['full_cache']).sum())} bytes differ"
    pn = p.np()
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    ref = O.prefill_attention(c["q"].float().numpy(), cu, c["full_cache"], c["bt"], np.asarray(ctx, np.int32), 4, D,
                              pn["kc"], pn["vc"], pn["R"], 1.0 / math.sqrt(D), "bfloat16")
    got = out.float().cpu().numpy()
    for name, rows in (("decodes", slice(0, 5)), ("chunks", slice(5, None))):
        err, excess, cs = check_tolerance(got[rows], ref[rows], "bfloat16", rot_block=p.blk)
        print(f"mixed {name}: max_abs={err:.3e} excess={excess:.3e} cos={cs:.6f}")
        assert excess <= 0 and cs >= 0.999, name


def test_backend_decode_step_graph_replay(monkeypatch):
    """One decode step through RQAttentionImpl.forward (compress + store of the new token,
    fused decode) captured in a HIP graph, as vLLM captures UNIFORM_SINGLE_TOKEN_DECODE
    batches.  Replays, with eager forwards in between -- one of them with a block table
    twice as wide, which grows the shared decode workspace past the captured buffer --
    reproduce the eager output bit for bit."""
    from rotorquant_vllm import kernels as K
    ctx = [700, 4000, 33, 2500]
    impl, p, c = _mixed_setup(monkeypatch, 8, 32, "iso", 3, "fast", ctx, [1, 1, 1, 1], 72)
    dev = torch.device("cuda")
    kv_cache = torch.from_numpy(c["cache0"]).to(dev)
    q, kn, vn = c["q"].to(dev), c["k_new"].to(dev), c["v_new"].to(dev)
    md = c["md"]
    out = torch.empty(q.shape, dtype=torch.bfloat16, device=dev)

    def step():
        impl.forward(None, q, kn, vn, kv_cache, md, output=out)

    step()
    torch.cuda.synchronize()
    eager = out.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    # an eager batch whose block table is wide enough that its tile descriptors outgrow
    # the decode workspace in use (sized at init, or grown by earlier calls)
    from rotorquant_vllm import _lib
    cur = K._ws_cache[(str(q.device), "decode")].numel()
    width = 1024
    while _lib.load().rq_fused_decode_workspace_bytes(4, 32, D, width * BS) <= cur:
        width *= 2
    wide_bt = torch.zeros(4, width, dtype=torch.int32, device=dev)
    wide_bt[:, :md.block_table.shape[1]] = md.block_table
    md_wide = _metadata(4, 1, md.slot_mapping.cpu().numpy(), wide_bt.cpu().numpy(), ctx, [1, 1, 1, 1])
    out_wide = torch.empty_like(out)
    n_retired = len(K._ws_retired)
    for i in range(3):
        out.zero_()
        impl.forward(None, q, kn, vn, kv_cache, md_wide, output=out_wide)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        assert torch.equal(out_wide, eager)
    assert len(K._ws_retired) > n_retired, "the wide batch should have grown the decode workspace"
    pn = p.np()
    ref = O.decode_attention(c["q"].float().numpy(), c["full_cache"], c["bt"], np.asarray(ctx, np.int32), 8, D,
                             pn["kc"], pn["vc"], pn["R"], 1.0 / math.sqrt(D), "bfloat16")
    _, excess, cs = check_tolerance(eager.float().cpu().numpy(), ref, "bfloat16", rot_block=p.blk)
    assert excess <= 0 and cs >= 0.999


def test_backend_unfused_mixed_batch_and_decode_graph(monkeypatch):
    """The default (non-fused) path: a mixed batch of decodes and chunks in one forward
    -- the decodes through the decode kernel, the two chunks through one
    rq_paged_prefill call -- checked against the oracle of the reference's non-fused
    path; then a decode step on the same path captured in a HIP graph replays the
    eager output bit for bit (no host read of the metadata; the decode workspace was
    allocated at the first forward)."""
    ctx = [3000, 700, 5, 800, 64]
    q_lens = [1, 1, 1, 200, 64]
    impl, p, c = _mixed_setup(monkeypatch, 4, 28, "iso", 3, "full", ctx, q_lens, 73, fused=False)
    assert not impl._fused_paged_available and not impl._fused_prefill_available
    import rotorquant_vllm.vllm.rq_backend as rq_backend_module
    seen = []

    def counted(name, fn):
        def wrapper(q, kv_cache, block_table, seq_lens, *a, **k):
            seen.append((name, seq_lens.shape[0]))
            return fn(q, kv_cache, block_table, seq_lens, *a, **k)
        return wrapper

    monkeypatch.setattr(rq_backend_module, "_paged_attention_fn",
                        counted("attention", rq_backend_module._paged_attention_fn))
    monkeypatch.setattr(rq_backend_module, "_paged_prefill_fn", counted("prefill", rq_backend_module._paged_prefill_fn))
    monkeypatch.setattr(rq_backend_module, "_unfused_decode_fn", counted("decode", rq_backend_module._unfused_decode_fn))
    dev = torch.device("cuda")
    kv_cache = torch.from_numpy(c["cache0"]).to(dev)
    out = torch.empty(c["q"].shape, dtype=torch.bfloat16, device=dev)
    impl.forward(None, c["q"].to(dev), c["k_new"].to(dev), c["v_new"].to(dev), kv_cache, c["md"], output=out)
    torch.cuda.synchronize()
    assert seen == [("decode", 3), ("prefill", 2)], seen
    got_cache = kv_cache.cpu().numpy()
    assert np.array_equal(got_cache, c["full_cache"]), f"{int((got_cache != c['full_cache']).sum())} bytes differ"
    pn = p.np()
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    ref = O.unfused_attention(c["q"].float().numpy(), cu, c["full_cache"], c["bt"], np.asarray(ctx, np.int32), 4, D,
                              pn["kc"], pn["vc"], pn["R"], 1.0 / math.sqrt(D), "bfloat16")
    err, excess, cs = check_tolerance(out.float().cpu().numpy(), ref, "bfloat16", rot_block=p.blk)
    print(f"unfused mixed: max_abs={err:.3e} excess={excess:.3e} cos={cs:.6f}")
    assert excess <= 0 and cs >= 0.999

    # decode step (one new token for each of the first three sequences), captured
    dctx = [3001, 701, 6]
    bt = c["bt"][:3]
    slots = [int(bt[b][(L - 1) // BS]) * BS + (L - 1) % BS for b, L in enumerate(dctx)]
    md = _metadata(3, 1, slots, np.ascontiguousarray(bt), dctx, [1, 1, 1])
    qd = torch.randn(3, 28, D, generator=gen(7306)).to(torch.bfloat16).to(dev)
    kn = torch.randn(3, 4, D, generator=gen(7307)).to(torch.bfloat16).to(dev)
    vn = torch.randn(3, 4, D, generator=gen(7308)).to(torch.bfloat16).to(dev)
    outd = torch.empty_like(qd)

    def step():
        impl.forward(None, qd, kn, vn, kv_cache, md, output=outd)

    step()
    torch.cuda.synchronize()
    eager = outd.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for i in range(3):
        outd.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(outd, eager), f"replay {i}"


def test_backend_unfused_prefill_groups(monkeypatch):
    """The non-fused path with a prefill workspace that holds one 800-token sequence's
    tile images (4 kv heads): the three decodes of a mixed batch go to the decode
    kernel, its two chunks to rq_paged_prefill in two calls, each with its own
    max_seq_len and its absolute query rows, and the whole output matches the oracle
    of the reference's non-fused path."""
    from rotorquant_vllm import _lib
    from rotorquant_vllm import kernels as K
    import rotorquant_vllm.vllm.rq_backend as rq_backend_module
    ctx = [3000, 700, 5, 800, 64]
    q_lens = [1, 1, 1, 200, 64]
    impl, p, c = _mixed_setup(monkeypatch, 4, 28, "iso", 3, "full", ctx, q_lens, 74, fused=False)
    dev = torch.device("cuda", torch.cuda.current_device())
    kv_cache = torch.from_numpy(c["cache0"]).to(dev)
    impl._init_cg_buffers(kv_cache, torch.bfloat16)
    budget = _lib.load().rq_paged_prefill_workspace_bytes(1, 4, 800)
    monkeypatch.setitem(K._ws_cache, (str(dev), "prefill"), torch.empty(budget, dtype=torch.uint8, device=dev))
    seen = []

    def counted(name, fn):
        def wrapper(q, kv, block_table, seq_lens, cu, max_q, *a, **k):
            seen.append((name, seq_lens.shape[0], int(max_q), k.get("max_seq_len")))
            return fn(q, kv, block_table, seq_lens, cu, max_q, *a, **k)
        return wrapper

    def counted_decode(fn):
        def wrapper(q, kv, block_table, seq_lens, *a, **k):
            seen.append(("decode", seq_lens.shape[0], q.shape[0], k.get("max_seq_len")))
            return fn(q, kv, block_table, seq_lens, *a, **k)
        return wrapper

    monkeypatch.setattr(rq_backend_module, "_paged_attention_fn",
                        counted("attention", rq_backend_module._paged_attention_fn))
    monkeypatch.setattr(rq_backend_module, "_paged_prefill_fn", counted("prefill", rq_backend_module._paged_prefill_fn))
    monkeypatch.setattr(rq_backend_module, "_unfused_decode_fn", counted_decode(rq_backend_module._unfused_decode_fn))
    out = torch.full(c["q"].shape, float("nan"), dtype=torch.bfloat16, device=dev)
    print(f"unfused prefill groups: ctx={ctx} q_lens={q_lens} workspace={budget} B", flush=True)
    impl.forward(None, c["q"].to(dev), c["k_new"].to(dev), c["v_new"].to(dev), kv_cache, c["md"], output=out)
    torch.cuda.synchronize()
    cap = c["md"].block_table.shape[1] * BS
    assert seen == [("decode", 3, 3, cap), ("prefill", 1, 200, 800), ("prefill", 1, 64, 64)], seen
    pn = p.np()
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    ref = O.unfused_attention(c["q"].float().numpy(), cu, c["full_cache"], c["bt"], np.asarray(ctx, np.int32), 4, D,
                              pn["kc"], pn["vc"], pn["R"], 1.0 / math.sqrt(D), "bfloat16")
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all(), "every query row is written"
    err, excess, cs = check_tolerance(got, ref, "bfloat16", rot_block=p.blk)
    print(f"unfused prefill groups: max_abs={err:.3e} excess={excess:.3e} cos={cs:.6f}", flush=True)
    assert excess <= 0 and cs >= 0.999


def test_backend_fused_prefill_groups(monkeypatch):
    """The fused path with an int8-prefill workspace that holds one 800-token sequence's
    tile images (4 kv heads): the decodes go to the fused decode, the two chunks to
    rq_int8_prefill in two calls, each with its own max_seq_len and its absolute query
    rows, and every row matches the prefill oracle."""
    from rotorquant_vllm import _lib
    from rotorquant_vllm import kernels as K
    import rotorquant_vllm.vllm.rq_backend as rq_backend_module
    ctx = [3000, 700, 5, 800, 64]
    q_lens = [1, 1, 1, 200, 64]
    impl, p, c = _mixed_setup(monkeypatch, 4, 28, "iso", 3, "full", ctx, q_lens, 75)
    assert impl._fused_paged_available and impl._fused_prefill_available
    dev = torch.device("cuda", torch.cuda.current_device())
    kv_cache = torch.from_numpy(c["cache0"]).to(dev)
    impl._init_cg_buffers(kv_cache, torch.bfloat16)
    budget = _lib.load().rq_int8_prefill_workspace_bytes(1, 4, 800)
    monkeypatch.setitem(K._ws_cache, (str(dev), "prefill"), torch.empty(budget, dtype=torch.uint8, device=dev))
    seen = []
    fn = rq_backend_module._fused_paged_rq_int8_prefill_fn

    def counted(*a, **k):
        seen.append((a[3].shape[0], k.get("max_q_len"), k.get("max_seq_len")))
        return fn(*a, **k)

    monkeypatch.setattr(rq_backend_module, "_fused_paged_rq_int8_prefill_fn", counted)
    out = torch.full(c["q"].shape, float("nan"), dtype=torch.bfloat16, device=dev)
    print(f"fused prefill groups: ctx={ctx} q_lens={q_lens} workspace={budget} B", flush=True)
    impl.forward(None, c["q"].to(dev), c["k_new"].to(dev), c["v_new"].to(dev), kv_cache, c["md"], output=out)
    torch.cuda.synchronize()
    assert seen == [(1, 200, 800), (1, 64, 64)], seen
    pn = p.np()
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    ref = O.prefill_attention(c["q"].float().numpy(), cu, c["full_cache"], c["bt"], np.asarray(ctx, np.int32), 4, D,
                              pn["kc"], pn["vc"], pn["R"], 1.0 / math.sqrt(D), "bfloat16")
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all(), "every query row is written"
    err, excess, cs = check_tolerance(got, ref, "bfloat16", rot_block=p.blk)
    print(f"fused prefill groups: max_abs={err:.3e} excess={excess:.3e} cos={cs:.6f}", flush=True)
    assert excess <= 0 and cs >= 0.999
