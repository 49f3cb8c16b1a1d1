"""Layout KATs of the reference, env parsing, and the C ABI surface (no GPU)."""
import os
import re

import pytest
import torch

from rotorquant_vllm import _lib
from rotorquant_vllm.vllm import rq_backend as B

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


class TestCacheLayout:
    """Reference KATs: tests/test_vllm_integration.py:44-62, tests/test_benchmarks.py:144-156."""

    def test_nibble_packed_size(self):
        assert B._rq_bytes_per_token_kv(128, 8) == 1088
        assert B._rq_padded_slot_bytes(128) == 256
        assert 8 * B._rq_padded_slot_bytes(128) == 2048

    def test_cache_shape(self):
        assert B.RQAttentionBackend.get_kv_cache_shape(100, 16, 8, 128) == (100, 16, 2048)
        assert B.RQAttentionBackend.get_kv_cache_shape(7, 16, 4, 128) == (7, 16, 1024)

    def test_page_size(self):
        spec = B.RQFullAttentionSpec(block_size=16, num_kv_heads=8, head_size=128, dtype=torch.uint8)
        assert spec.real_page_size_bytes == 32768

    def test_compression_ratio(self):
        r = 8 * 128 * 2 * 2 / B._rq_bytes_per_token_kv(128, 8)
        assert 3.5 < r < 4.0

    def test_oracle_layout_agrees(self):
        import oracle as O
        lay = O.slot_layout(8, 128)
        assert lay == dict(k_idx_end=512, k_norm_end=544, v_idx_end=1056, v_norm_end=1088, total_bytes=2048,
                           index_bytes=64)


class TestEnv:
    def test_defaults(self, monkeypatch):
        for k in ("RQ_MODE", "RQ_BITS", "RQ_K_BITS", "RQ_V_BITS", "RQ_ISO_MODE", "RQ_USE_FUSED_PAGED"):
            monkeypatch.delenv(k, raising=False)
        assert B._parse_rq_mode() == "iso" and B._parse_iso_mode() == "fast"
        assert B._parse_kv_bits() == (3, 3) and B._parse_rq_fused_paged_env() is False

    def test_overrides(self, monkeypatch):
        monkeypatch.setenv("RQ_MODE", "PLANAR")
        monkeypatch.setenv("RQ_BITS", "4")
        monkeypatch.setenv("RQ_V_BITS", "3")
        monkeypatch.setenv("RQ_K_BITS", "")
        monkeypatch.setenv("RQ_USE_FUSED_PAGED", "Yes")
        assert B._parse_rq_mode() == "planar" and B._parse_kv_bits() == (4, 3)
        assert B._parse_rq_fused_paged_env() is True

    @pytest.mark.parametrize("var,val,msg", [
        ("RQ_MODE", "turbo", "RQ_MODE must be 'iso' or 'planar', got 'turbo'"),
        ("RQ_BITS", "2", "RQ_BITS must be 3 or 4, got '2'"),
        ("RQ_K_BITS", "5", "RQ_K_BITS must be 3 or 4, got '5'"),
        ("RQ_V_BITS", "8", "RQ_V_BITS must be 3 or 4, got '8'"),
        ("RQ_ISO_MODE", "slow", "RQ_ISO_MODE must be 'fast' or 'full', got 'slow'"),
    ])
    def test_invalid_values_raise(self, monkeypatch, var, val, msg):
        monkeypatch.setenv(var, val)
        fn = {"RQ_MODE": B._parse_rq_mode, "RQ_BITS": B._parse_rq_bits, "RQ_K_BITS": B._parse_kv_bits,
              "RQ_V_BITS": B._parse_kv_bits, "RQ_ISO_MODE": B._parse_iso_mode}[var]
        with pytest.raises(ValueError, match=re.escape(msg)):
            fn()


def _header_symbols():
    txt = open(os.path.join(ROOT, "include", "rq_abi.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char \*)\s*(rq_\w+)\(", txt, re.M)))


class TestABI:
    def test_library_exports_every_declared_symbol(self):
        lib = _lib.load()
        syms = _header_symbols()
        assert len(syms) >= 10
        for s in syms:
            assert hasattr(lib, s), s
        assert set(syms) == set(_lib.EXPORTED)

    def test_version(self):
        assert _lib.load().rq_abi_version() == 7

    def test_argument_validation_without_gpu(self):
        """Bad arguments are rejected before any device work, with a message."""
        lib = _lib.load()
        rc = lib.rq_compress(None, 7, 1, 128, None, None, 4, None, 7, None, None, None)
        assert rc == 1 and b"dtype" in lib.rq_last_error()
        rc = lib.rq_compress(None, 0, 1, 100, None, None, 4, None, 7, None, None, None)
        assert rc == 1 and b"head_dim" in lib.rq_last_error()
        rc = lib.rq_fused_decode(None, 1, 1, 32, 0, 0, None, 1, 16, 0, 0, 8, 64, 0, None, 1, 1, None, 16, None, 8,
                                 None, 8, None, 4, 0.1, None, 0, 0, None, 0, None)
        assert rc == 1 and b"head_dim" in lib.rq_last_error()
        rc = lib.rq_fused_decode(None, 1, 1, 40, 0, 0, None, 1, 16, 0, 0, 2, 128, 0, None, 1, 1, None, 16, None, 8,
                                 None, 8, None, 4, 0.1, None, 0, 0, None, 0, None)
        assert rc == 1 and b"integer <= 16" in lib.rq_last_error()
        # the dense 3-bit layout takes 8-entry codebooks only
        rc = lib.rq_fused_decode(None, 1, 1, 32, 0, 0, None, 1, 16, 0, 0, 8, 128, 1, None, 1, 1, None, 16, None, 16,
                                 None, 8, None, 4, 0.1, None, 0, 0, None, 0, None)
        assert rc == 1 and b"dense" in lib.rq_last_error()
        # rq_paged_attention: head_dim, GQA width, rotation block, centroid count
        base = dict(q=None, dtype=1, total_q=1, hq=32, qst=0, qsh=0, cu=None, ns=1, mq=1, causal=1, kv=None, nb=1,
                    bs=16, sb=0, st=0, h=8, d=128, il=0, bt=None, mb=1, bss=1, sl=None, kc=None, nk=8, vc=None,
                    nv=8, r=None, rb=4, sm=0.1, out=None, ost=0, osh=0, stream=None)
        for change, msg in ((dict(d=64), b"head_dim"), (dict(hq=136), b"integer <= 16"), (dict(rb=8), b"rot_block"),
                            (dict(nk=17), b"centroid"), (dict(dtype=2), b"dtype"), (dict(il=1, nv=16), b"dense"),
                            (dict(il=2), b"index_layout")):
            rc = lib.rq_paged_attention(*{**base, **change}.values())
            assert rc == 1 and msg in lib.rq_last_error(), change
        # rq_paged_prefill: the same checks, plus its workspace (none given here)
        pre = {k: v for k, v in base.items() if k != "stream"}
        pre = {**{k: pre[k] for k in list(pre)[:list(pre).index("sl") + 1]}, "msl": 16,
               **{k: pre[k] for k in list(pre)[list(pre).index("sl") + 1:]}, "ws": None, "wsb": 0, "stream": None}
        for change, msg in ((dict(d=64), b"head_dim"), (dict(hq=136), b"integer <= 16"), (dict(rb=8), b"rot_block"),
                            (dict(nk=17), b"centroid"), (dict(dtype=2), b"dtype"), (dict(il=1, nv=16), b"dense"),
                            (dict(il=2), b"index_layout"), (dict(msl=-1), b"bad sizes")):
            rc = lib.rq_paged_prefill(*{**pre, **change}.values())
            assert rc == 1 and msg in lib.rq_last_error(), change
        # a workspace smaller than the call needs: RQ_ENOSPACE (2); a missing one: RQ_EINVAL
        assert lib.rq_paged_prefill(*pre.values()) == 2 and b"workspace too small" in lib.rq_last_error()
        assert lib.rq_paged_prefill(*{**pre, "wsb": 1 << 30}.values()) == 1 and b"aligned" in lib.rq_last_error()
        rc = lib.rq_fused_decode(None, 1, 1, 32, 0, 0, None, 1, 16, 0, 0, 8, 128, 0, None, 1, 1, None, 16, None, 8,
                                 None, 8, None, 4, 0.1, None, 0, 0, None, 0, None)
        assert rc == 2 and b"workspace too small" in lib.rq_last_error()
        assert lib.rq_paged_prefill(*{**pre, "msl": 0}.values()) == 0  # nothing to attend: no launch
        assert lib.rq_paged_prefill_workspace_bytes(3, 8, 1000) == lib.rq_int8_prefill_workspace_bytes(3, 8, 1000)
        with pytest.raises(ValueError):
            _lib.check(1, "x")

    def test_kernels_reject_cpu_tensors(self):
        from rotorquant_vllm import kernels as K
        with pytest.raises(RuntimeError, match="no CPU path"):
            K.iso_decompress(torch.zeros(1, 1, 64, dtype=torch.uint8), torch.ones(1, 1, 1), torch.zeros(8),
                             torch.float16)


def test_rotation_block_cache_is_per_tensor_object():
    """Two tensor objects over the same memory (as when a freed R's memory is reused
    by the next one) each get their own block width: the cache is keyed by the
    tensor object, not by its address."""
    from rotorquant_vllm import kernels as K
    from rq_testlib import Params
    iso, planar = Params("iso", 3, 3).R, Params("planar", 3, 3).R
    s = torch.zeros(128 * 128)
    s.numpy()[:] = planar.numpy().ravel()  # written behind torch's version counter
    a = s.view(128, 128)
    assert K.rotation_block(a) == 2
    s.numpy()[:] = iso.numpy().ravel()
    b = s.view(128, 128)
    assert b.data_ptr() == a.data_ptr() and b._version == a._version
    assert K.rotation_block(b) == 4
