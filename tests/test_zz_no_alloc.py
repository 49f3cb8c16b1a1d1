"""rq_fused_decode_noalloc (static scratch, no workspace argument) against rq_fused_decode.

Both entry points are called through the C ABI (ctypes) on the same inputs:
the outputs must agree bit for bit (same kernels and grid; only the scratch
address differs), on two calls in a row -- the second on a smaller batch, so
the static scratch holds the first call's larger contents when the second one
runs -- and a call needing more scratch than RQ_DECODE_SCRATCH_BYTES must be
refused with RQ_ENOSPACE before anything is launched.
"""
import pytest
import torch

from rq_testlib import decode_case

pytestmark = pytest.mark.gpu

RQ_ENOSPACE = 2
SCRATCH_BYTES = 256 << 20  # RQ_DECODE_SCRATCH_BYTES in include/rq_abi.h


def _args(case, dev):
    """Argument tuple shared by both entry points (everything but the workspace);
    index layout 0 (nibbles)."""
    from rotorquant_vllm import _lib
    p = case["p"]
    t = dict(q=case["q"].to(dev), cache=torch.from_numpy(case["cache"]).to(dev),
             bt=torch.from_numpy(case["bt"]).to(dev), sl=torch.from_numpy(case["lens"]).to(dev),
             kc=p.kc.to(dev), vc=p.vc.to(dev), R=p.R.to(dev))
    t["out"] = torch.empty_like(t["q"])
    B, HQ, D = t["q"].shape
    NB, BS, _ = t["cache"].shape
    max_len = int(case["lens"].max())
    head = (t["q"].data_ptr(), _lib.DTYPE_BF16, B, HQ, t["q"].stride(0), t["q"].stride(1), t["cache"].data_ptr(), NB,
            BS, t["cache"].stride(0), t["cache"].stride(1), case["H"], D, 0, t["bt"].data_ptr(), t["bt"].shape[1],
            t["bt"].stride(0), t["sl"].data_ptr(), max_len, t["kc"].data_ptr(), 8, t["vc"].data_ptr(), 8,
            t["R"].data_ptr(), p.blk, float(case["sm_scale"]))
    return t, head, max_len


def _run_both(case):
    from rotorquant_vllm import _lib
    L = _lib.load()
    dev = torch.device("cuda")
    stream = _lib.stream_ptr(dev)
    t, head, max_len = _args(case, dev)
    B, HQ, D = t["q"].shape
    out_ref = torch.empty_like(t["out"])
    ws = torch.empty(L.rq_fused_decode_workspace_bytes(B, HQ, D, max_len), dtype=torch.uint8, device=dev)
    _lib.check(L.rq_fused_decode(*head, out_ref.data_ptr(), out_ref.stride(0), out_ref.stride(1), ws.data_ptr(),
                                 ws.numel(), stream), "rq_fused_decode")
    _lib.check(L.rq_fused_decode_noalloc(*head, t["out"].data_ptr(), t["out"].stride(0), t["out"].stride(1),
                                         stream), "rq_fused_decode_noalloc")
    torch.cuda.synchronize()
    return t["out"].cpu(), out_ref.cpu()


def test_noalloc_matches_workspace_entry_point_twice():
    big = decode_case(81, 24, 8, 32, [7000, 1, 33, 4096] * 6)
    small = decode_case(82, 3, 8, 32, [300, 17, 2])
    for tag, case in (("first (24 sequences)", big), ("second (3 sequences)", small)):
        print(f"no-alloc decode, {tag}", flush=True)
        got, ref = _run_both(case)
        assert torch.equal(got, ref), tag
        assert torch.isfinite(got.float()).all()


def test_noalloc_refuses_oversize_without_launch():
    """A batch whose scratch need exceeds the static array is refused (RQ_ENOSPACE)."""
    from rotorquant_vllm import _lib
    L = _lib.load()
    case = decode_case(83, 2, 8, 32, [64, 10])
    dev = torch.device("cuda")
    t, head, _ = _args(case, dev)
    head = list(head)
    huge = 1 << 26  # 67 M tokens of max_seq_len: tile descriptors alone need > 256 MiB
    assert L.rq_fused_decode_workspace_bytes(2, 32, 128, huge) > SCRATCH_BYTES
    head[18] = huge           # max_seq_len
    head[15] = huge // 16     # max_blocks (the table is not read: the call is refused first)
    t["out"].fill_(1.5)  # a known value (an empty tensor may hold NaN bit patterns, which never compare equal)
    sentinel = t["out"].clone()
    rc = L.rq_fused_decode_noalloc(*head, t["out"].data_ptr(), t["out"].stride(0), t["out"].stride(1),
                                   _lib.stream_ptr(dev))
    torch.cuda.synchronize()
    assert rc == RQ_ENOSPACE
    assert b"scratch" in L.rq_last_error()
    assert torch.equal(t["out"], sentinel)
