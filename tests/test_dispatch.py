"""Dispatch plumbing of RQAttentionImpl.forward with fake kernels (CPU, no GPU, no vLLM).

The first two tests re-create the reference's TestFusedDecodeSelection
(tests/test_vllm_integration.py:109-239) against this build: the impl is made
with __new__, the private attributes the reference sets are set, and the
module-level kernel hooks are replaced by fakes with the reference's own
signatures (no keyword beyond sm_scale / out).  The remaining tests cover what
this build adds around the same hooks: the mixed-batch split (leading decodes
to the fused decode, the rest to the int8 prefill in workspace-bounded
groups), the shape gate of the fused kernels, the import-path alias and the
shared workspaces' lifetime.
"""
from types import SimpleNamespace

import pytest
import torch

import rotorquant_vllm.vllm.rq_backend as rq_backend_module
from rotorquant_vllm.vllm.rq_backend import AttentionType, RQAttentionImpl


def _bare_impl(fused_decode: bool, fused_prefill: bool):
    impl = RQAttentionImpl.__new__(RQAttentionImpl)
    impl.attn_type = AttentionType.DECODER
    impl._cg_buffers_ready = True
    impl._fused_paged_available = fused_decode
    impl._fused_prefill_available = fused_prefill
    impl.num_kv_heads = 8
    impl.head_size = 128
    impl.block_size = 16
    impl.scale = 0.125
    impl._k_quantizer = SimpleNamespace(centroids=torch.randn(16, dtype=torch.float32))
    impl._v_quantizer = SimpleNamespace(centroids=torch.randn(16, dtype=torch.float32))
    impl._rq_rot = torch.eye(128, dtype=torch.float32)
    return impl


class TestFusedDecodeSelection:
    """The reference's two fake-based tests, unchanged in substance."""

    def test_decode_uses_fused_kernel_when_enabled(self, monkeypatch):
        impl = _bare_impl(True, False)
        called = {}

        def fake_fused(q, kv_cache, block_table, seq_lens, centroids_k, centroids_v, rotation,
                       num_kv_heads, head_dim, block_size, sm_scale=None, out=None):
            called["q_shape"] = tuple(q.shape)
            called["kv_shape"] = tuple(kv_cache.shape)
            called["block_table_shape"] = tuple(block_table.shape)
            called["seq_lens"] = seq_lens.clone()
            called["num_kv_heads"] = num_kv_heads
            called["head_dim"] = head_dim
            called["block_size"] = block_size
            called["sm_scale"] = sm_scale
            out.fill_(3.0)
            return out

        monkeypatch.setattr(rq_backend_module, "_fused_paged_rq_decode_fn", fake_fused)
        query = torch.randn(1, 8, 128, dtype=torch.bfloat16)
        kv_cache = torch.zeros(4, 16, 2048, dtype=torch.uint8)
        output = torch.zeros_like(query)
        md = SimpleNamespace(num_actual_tokens=1, block_table=torch.zeros(1, 4, dtype=torch.int32),
                             seq_lens=torch.tensor([1], dtype=torch.int32))
        result = impl.forward(layer=None, query=query, key=None, value=None, kv_cache=kv_cache, attn_metadata=md,
                              output=output)
        assert result is output
        assert torch.all(output == 3.0)
        assert called == {"q_shape": (1, 8, 128), "kv_shape": (4, 16, 2048), "block_table_shape": (1, 4),
                          "seq_lens": torch.tensor([1], dtype=torch.int32), "num_kv_heads": 8, "head_dim": 128,
                          "block_size": 16, "sm_scale": 0.125}

    def test_prefill_uses_fused_int8_kernel_when_enabled(self, monkeypatch):
        impl = _bare_impl(False, True)
        called = {}

        def fake_prefill(q, kv_cache, block_table, seq_lens, centroids_k, centroids_v, rotation,
                         num_kv_heads, head_dim, block_size, sm_scale=None, out=None):
            called["q_shape"] = tuple(q.shape)
            called["kv_shape"] = tuple(kv_cache.shape)
            called["block_table_shape"] = tuple(block_table.shape)
            called["seq_lens"] = seq_lens.clone()
            called["num_kv_heads"] = num_kv_heads
            called["head_dim"] = head_dim
            called["block_size"] = block_size
            called["sm_scale"] = sm_scale
            out.fill_(5.0)
            return out

        monkeypatch.setattr(rq_backend_module, "_fused_paged_rq_int8_prefill_fn", fake_prefill)
        query = torch.randn(3, 8, 128, dtype=torch.bfloat16)
        kv_cache = torch.zeros(4, 16, 2048, dtype=torch.uint8)
        output = torch.zeros_like(query)
        md = SimpleNamespace(num_actual_tokens=3, block_table=torch.zeros(1, 4, dtype=torch.int32),
                             seq_lens=torch.tensor([3], dtype=torch.int32), use_cascade=False,
                             slot_mapping=torch.arange(3, dtype=torch.int64))
        result = impl.forward(layer=None, query=query, key=None, value=None, kv_cache=kv_cache, attn_metadata=md,
                              output=output)
        assert result is output
        assert torch.all(output == 5.0)
        assert called == {"q_shape": (3, 8, 128), "kv_shape": (4, 16, 2048), "block_table_shape": (1, 4),
                          "seq_lens": torch.tensor([3], dtype=torch.int32), "num_kv_heads": 8, "head_dim": 128,
                          "block_size": 16, "sm_scale": 0.125}


def _mixed_metadata(q_lens, seq_lens, max_blocks=64, host_copies=True):
    cu = torch.tensor([0] + list(torch.tensor(q_lens).cumsum(0).tolist()), dtype=torch.int32)
    md = SimpleNamespace(num_actual_tokens=int(sum(q_lens)), max_query_len=max(q_lens), use_cascade=False,
                         block_table=torch.arange(len(q_lens) * max_blocks, dtype=torch.int32).reshape(-1, max_blocks),
                         seq_lens=torch.tensor(seq_lens, dtype=torch.int32), query_start_loc=cu,
                         slot_mapping=torch.arange(int(sum(q_lens)), dtype=torch.int64))
    if host_copies:
        md.rq_query_start_loc_cpu = cu.clone()
        md.rq_seq_lens_cpu = md.seq_lens.clone()
    return md


@pytest.mark.parametrize("host_copies", [True, False])
def test_mixed_batch_splits_decodes_and_prefill_groups(monkeypatch, host_copies):
    """[3 decodes | 3 chunks]: one decode call on sequences 0..2 (query rows 0..2), then
    int8 prefill calls over contiguous ranges of the chunks whose tile images fit the
    prefill workspace (here sized for 2 x 320 keys x 8 kv heads); every query row is
    written exactly once, by the call that owns its sequence."""
    from rotorquant_vllm import _lib
    from rotorquant_vllm import kernels as K
    impl = _bare_impl(True, True)
    calls = []

    def fake_decode(q, kv_cache, block_table, seq_lens, centroids_k, centroids_v, rotation, num_kv_heads, head_dim,
                    block_size, sm_scale=None, out=None, max_seq_len=None, workspace=None):
        calls.append(("decode", tuple(q.shape), seq_lens.tolist(), tuple(block_table.shape), max_seq_len))
        out.add_(1.0)
        return out

    def fake_prefill(q, kv_cache, block_table, seq_lens, centroids_k, centroids_v, rotation, num_kv_heads, head_dim,
                     block_size, sm_scale=None, out=None, cu_seqlens_q=None, max_q_len=None, max_seq_len=None,
                     workspace=None):
        calls.append(("prefill", seq_lens.tolist(), cu_seqlens_q.tolist(), max_q_len, max_seq_len))
        cu = cu_seqlens_q.tolist()
        out[cu[0]:cu[-1]] += 1.0
        return out

    monkeypatch.setattr(rq_backend_module, "_fused_paged_rq_decode_fn", fake_decode)
    monkeypatch.setattr(rq_backend_module, "_fused_paged_rq_int8_prefill_fn", fake_prefill)
    budget = _lib.load().rq_int8_prefill_workspace_bytes(2, 8, 320)
    monkeypatch.setitem(K._ws_cache, ("cpu", "prefill"), torch.empty(budget, dtype=torch.uint8))
    q_lens, seq_lens = [1, 1, 1, 40, 7, 100], [500, 30, 9, 300, 107, 320]
    md = _mixed_metadata(q_lens, seq_lens, host_copies=host_copies)
    query = torch.randn(md.num_actual_tokens, 8, 128)
    output = torch.zeros_like(query)
    impl.forward(None, query, None, None, torch.zeros(40, 16, 2048, dtype=torch.uint8), md, output=output)
    assert calls[0] == ("decode", (3, 8, 128), [500, 30, 9], (3, 64), 64 * 16)
    assert calls[1:] == [("prefill", [300, 107], [3, 43, 50], 40, 300), ("prefill", [320], [50, 150], 100, 320)]
    assert torch.all(output == 1.0)


def test_mixed_batch_with_reference_signature_prefill_hook(monkeypatch):
    """A prefill hook with the reference's signature (one sequence, no cu_seqlens_q) on a
    mixed batch [1, 1, 1, 40 | 7]: it is called once per multi-token sequence with that
    sequence's own query / output rows, block-table row and length; the decode rows are
    written only by the decode hook."""
    impl = _bare_impl(True, True)
    calls = []

    def fake_decode(q, kv_cache, block_table, seq_lens, centroids_k, centroids_v, rotation, num_kv_heads, head_dim,
                    block_size, sm_scale=None, out=None):
        calls.append(("decode", tuple(q.shape), seq_lens.tolist()))
        out.fill_(1.0)
        return out

    def fake_prefill(q, kv_cache, block_table, seq_lens, centroids_k, centroids_v, rotation, num_kv_heads, head_dim,
                     block_size, sm_scale=None, out=None):
        if seq_lens.numel() != 1:
            raise ValueError("single sequence only")
        calls.append(("prefill", tuple(q.shape), seq_lens.tolist(), block_table[0, 0].item()))
        out.fill_(7.0)
        return out

    monkeypatch.setattr(rq_backend_module, "_fused_paged_rq_decode_fn", fake_decode)
    monkeypatch.setattr(rq_backend_module, "_fused_paged_rq_int8_prefill_fn", fake_prefill)
    q_lens, seq_lens = [1, 1, 1, 40, 7], [300, 30, 9, 300, 107]
    md = _mixed_metadata(q_lens, seq_lens)
    query = torch.randn(md.num_actual_tokens, 8, 128)
    output = torch.zeros_like(query)
    impl.forward(None, query, None, None, torch.zeros(40, 16, 2048, dtype=torch.uint8), md, output=output)
    assert calls == [("decode", (3, 8, 128), [300, 30, 9]), ("prefill", (40, 8, 128), [300], 3 * 64),
                     ("prefill", (7, 8, 128), [107], 4 * 64)]
    assert torch.all(output[:3] == 1.0) and torch.all(output[3:] == 7.0)


def test_single_token_batch_goes_to_decode_only(monkeypatch):
    impl = _bare_impl(True, True)
    seen = []
    monkeypatch.setattr(rq_backend_module, "_fused_paged_rq_decode_fn",
                        lambda q, *a, out=None, **k: seen.append(("decode", q.shape[0])) or out)
    monkeypatch.setattr(rq_backend_module, "_fused_paged_rq_int8_prefill_fn",
                        lambda *a, **k: seen.append("prefill"))
    md = _mixed_metadata([1, 1, 1, 1], [10, 20, 30, 40])
    q = torch.randn(4, 8, 128)
    impl.forward(None, q, None, None, torch.zeros(8, 16, 2048, dtype=torch.uint8), md, output=torch.zeros_like(q))
    assert seen == [("decode", 4)]


def test_fused_flags_follow_the_kernel_shapes(monkeypatch):
    """RQ_USE_FUSED_PAGED=1 turns the fused paths on only for shapes the kernels take:
    head_size 128 and a GQA group <= 16 (a head_size 64 model keeps the unfused path)."""
    monkeypatch.setenv("RQ_USE_FUSED_PAGED", "1")
    monkeypatch.setenv("RQ_MODE", "planar")
    monkeypatch.setenv("RQ_BITS", "3")
    for num_heads, num_kv, head_size, on in ((32, 8, 128, True), (32, 8, 64, False), (32, 1, 128, False),
                                             (28, 4, 128, True)):
        impl = RQAttentionImpl(num_heads, head_size, head_size ** -0.5, num_kv_heads=num_kv)
        assert impl._fused_paged_available == on and impl._fused_prefill_available == on, (num_heads, num_kv,
                                                                                          head_size)
    spec = SimpleNamespace(head_size=64)
    assert (rq_backend_module.RQMetadataBuilder.get_cudagraph_support(None, spec)
            == rq_backend_module.AttentionCGSupport.NEVER)
    spec = SimpleNamespace(head_size=128)
    assert (rq_backend_module.RQMetadataBuilder.get_cudagraph_support(None, spec)
            == rq_backend_module.AttentionCGSupport.UNIFORM_SINGLE_TOKEN_DECODE)
    # shapes or dtypes whose decodes run the torch fallback (not capturable): NEVER
    for num_heads, dtype, exp in ((32, torch.bfloat16, "UNIFORM_SINGLE_TOKEN_DECODE"), (32, torch.float32, "NEVER"),
                                  (8 * 17, torch.float16, "NEVER")):
        mc = SimpleNamespace(dtype=dtype, get_num_attention_heads=lambda pc, n=num_heads: n)
        cfg = SimpleNamespace(model_config=mc, parallel_config=None)
        spec = SimpleNamespace(head_size=128, num_kv_heads=8)
        got = rq_backend_module.RQMetadataBuilder.get_cudagraph_support(cfg, spec)
        assert got == getattr(rq_backend_module.AttentionCGSupport, exp), (num_heads, dtype)


def test_triton_import_path_is_the_hip_op():
    import rotorquant_vllm.kernels as K
    from rotorquant_vllm.triton import (fused_paged_rq_decode, fused_paged_rq_int8_prefill, iso_compress,
                                        iso_decompress, planar_compress, planar_decompress)
    assert fused_paged_rq_decode is K.fused_paged_rq_decode
    assert fused_paged_rq_int8_prefill is K.fused_paged_rq_int8_prefill
    assert (iso_compress, iso_decompress, planar_compress, planar_decompress) == (
        K.iso_compress, K.iso_decompress, K.planar_compress, K.planar_decompress)


def test_workspace_growth_keeps_captured_buffers_alive(monkeypatch):
    """A call that needs more scratch than the buffer a HIP graph captured gets a new
    buffer; the captured one stays allocated (its address stays valid for replays)."""
    from rotorquant_vllm import kernels as K
    monkeypatch.setattr(K, "_ws_cache", {})
    monkeypatch.setattr(K, "_ws_retired", [])
    small = K.shared_workspace("cpu", "decode", 1000)
    ptr = small.data_ptr()
    assert K.shared_workspace("cpu", "decode", 500) is small      # fits: same buffer
    big = K.shared_workspace("cpu", "decode", 5000)               # grows
    assert big is not small and big.numel() >= 5000
    assert any(t.data_ptr() == ptr for t in K._ws_retired)        # the old one is still held
    assert K.shared_workspace("cpu", "decode", 4000) is big


@pytest.mark.parametrize("causal", [True, False])
def test_unfused_short_queries_are_one_paged_attention_call(monkeypatch, causal):
    """Without RQ_USE_FUSED_PAGED a batch whose queries are all short (at most
    RQ_UNFUSED_SHORT_Q tokens) is one rq_paged_attention call over the whole batch,
    with vLLM's device metadata as is (no host copies read) and max_query_len /
    causal from the metadata."""
    impl = _bare_impl(False, False)
    calls = []

    def fake(q, kv_cache, block_table, seq_lens, cu_seqlens_q, max_q_len, kc, vc, R, num_kv_heads, head_dim,
             block_size, sm_scale=None, causal=True, out=None):
        calls.append((tuple(q.shape), block_table is md.block_table, seq_lens is md.seq_lens,
                      cu_seqlens_q is md.query_start_loc, max_q_len, causal, num_kv_heads, head_dim, block_size,
                      sm_scale))
        out.fill_(2.0)
        return out

    def no_prefill(*a, **k):
        raise AssertionError("short queries must not reach rq_paged_prefill")

    monkeypatch.setattr(rq_backend_module, "_paged_attention_fn", fake)
    monkeypatch.setattr(rq_backend_module, "_paged_prefill_fn", no_prefill)
    md = _mixed_metadata([1, 1, 16, 7], [500, 30, 300, 107], host_copies=False)
    md.causal = causal
    query = torch.randn(md.num_actual_tokens + 3, 32, 128, dtype=torch.bfloat16)  # 3 padding rows
    output = torch.zeros_like(query)
    impl.forward(None, query, None, None, torch.zeros(40, 16, 2048, dtype=torch.uint8), md, output=output)
    assert rq_backend_module.RQ_UNFUSED_SHORT_Q == 16
    assert calls == [((25, 32, 128), True, True, True, 16, causal, 8, 128, 16, 0.125)]
    assert torch.all(output[:25] == 2.0) and torch.all(output[25:] == 0.0)


@pytest.mark.parametrize("causal", [True, False])
def test_unfused_long_queries_split_to_paged_prefill(monkeypatch, causal):
    """A non-fused batch with a query longer than RQ_UNFUSED_SHORT_Q: its leading
    single-token decode (sequence 0) goes to the decode kernel, the following short
    query (sequence 1) to one rq_paged_attention call, the rest to rq_paged_prefill in
    contiguous groups whose tile images fit the prefill workspace (sized here for 2 x
    320 keys x 8 kv heads), each with its own max_seq_len and max_q_len; every query
    row is written exactly once."""
    from rotorquant_vllm import _lib
    from rotorquant_vllm import kernels as K
    impl = _bare_impl(False, False)
    calls = []

    def fake_decode(q, kv_cache, block_table, seq_lens, centroids_k, centroids_v, rotation, num_kv_heads, head_dim,
                    block_size, sm_scale=None, out=None, max_seq_len=None, workspace=None):
        calls.append(("decode", tuple(q.shape), seq_lens.tolist(), tuple(block_table.shape), max_seq_len))
        out += 1.0
        return out

    def fake_attn(q, kv_cache, block_table, seq_lens, cu_seqlens_q, max_q_len, kc, vc, R, num_kv_heads, head_dim,
                  block_size, sm_scale=None, causal=True, out=None):
        calls.append(("attn", seq_lens.tolist(), cu_seqlens_q.tolist(), tuple(block_table.shape), max_q_len, causal))
        cu = cu_seqlens_q.tolist()
        out[cu[0]:cu[-1]] += 1.0
        return out

    def fake_prefill(q, kv_cache, block_table, seq_lens, cu_seqlens_q, max_q_len, kc, vc, R, num_kv_heads, head_dim,
                     block_size, sm_scale=None, causal=True, out=None, max_seq_len=None, workspace=None):
        calls.append(("prefill", seq_lens.tolist(), cu_seqlens_q.tolist(), max_q_len, max_seq_len, causal))
        cu = cu_seqlens_q.tolist()
        out[cu[0]:cu[-1]] += 1.0
        return out

    monkeypatch.setattr(rq_backend_module, "_paged_attention_fn", fake_attn)
    monkeypatch.setattr(rq_backend_module, "_paged_prefill_fn", fake_prefill)
    monkeypatch.setattr(rq_backend_module, "_unfused_decode_fn", fake_decode)
    budget = _lib.load().rq_paged_prefill_workspace_bytes(2, 8, 320)
    monkeypatch.setitem(K._ws_cache, ("cpu", "prefill"), torch.empty(budget, dtype=torch.uint8))
    q_lens, seq_lens = [1, 3, 40, 7, 100], [500, 30, 300, 107, 320]
    md = _mixed_metadata(q_lens, seq_lens)
    md.causal = causal
    query = torch.randn(md.num_actual_tokens, 32, 128, dtype=torch.float16)
    output = torch.zeros_like(query)
    impl.forward(None, query, None, None, torch.zeros(40, 16, 2048, dtype=torch.uint8), md, output=output)
    assert calls == [("decode", (1, 32, 128), [500], (1, 64), 64 * 16),
                     ("attn", [30], [1, 4], (1, 64), 3, causal),
                     ("prefill", [300, 107], [4, 44, 51], 40, 300, causal),
                     ("prefill", [320], [51, 151], 100, 320, causal)]
    assert torch.all(output == 1.0)


@pytest.mark.parametrize("causal", [True, False])
def test_unfused_decode_batch_takes_the_decode_kernel(monkeypatch, causal):
    """Without RQ_USE_FUSED_PAGED a uniform batch of single-token decodes
    (max_query_len 1) is one decode-kernel call (rq_fused_decode: the same K/V
    rounding and exact products as rq_paged_attention) with the block table's
    capacity as max_seq_len and no host read of the metadata; the fused path's hook
    _fused_paged_rq_decode_fn is not used."""
    impl = _bare_impl(False, False)
    calls = []

    def fake_decode(q, kv_cache, block_table, seq_lens, centroids_k, centroids_v, rotation, num_kv_heads, head_dim,
                    block_size, sm_scale=None, out=None, max_seq_len=None, workspace=None):
        calls.append((tuple(q.shape), block_table is md.block_table, seq_lens is md.seq_lens, max_seq_len, sm_scale))
        out.fill_(4.0)
        return out

    def unused(*a, **k):
        raise AssertionError("a decode batch must not reach this kernel")

    monkeypatch.setattr(rq_backend_module, "_unfused_decode_fn", fake_decode)
    monkeypatch.setattr(rq_backend_module, "_fused_paged_rq_decode_fn", unused)
    monkeypatch.setattr(rq_backend_module, "_paged_attention_fn", unused)
    monkeypatch.setattr(rq_backend_module, "_paged_prefill_fn", unused)
    md = _mixed_metadata([1, 1, 1, 1], [500, 30, 300, 107], host_copies=False)
    md.causal = causal
    query = torch.randn(4 + 2, 32, 128, dtype=torch.bfloat16)  # 2 padding rows
    output = torch.zeros_like(query)
    impl.forward(None, query, None, None, torch.zeros(40, 16, 2048, dtype=torch.uint8), md, output=output)
    assert calls == [((4, 32, 128), True, True, 64 * 16, 0.125)]
    assert torch.all(output[:4] == 4.0) and torch.all(output[4:] == 0.0)
