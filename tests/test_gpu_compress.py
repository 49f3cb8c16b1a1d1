"""GPU parity: compress / decompress / compress_store / paged decompress vs the CPU oracle.

Bit-exact: packed indices, fp32 norm bytes, decompressed values and every
byte of every written cache slot (padding included).
"""
import numpy as np
import pytest
import torch

import oracle as O
from rq_testlib import Params, build_cache_oracle, kv_config0, paged_layout

pytestmark = pytest.mark.gpu

GOLDEN = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "golden_cpu.npz"))


def _kernels():
    from rotorquant_vllm import kernels
    return kernels


def _dev(t):
    return t.to("cuda")


@pytest.mark.parametrize("mode", ["iso_fast", "iso_full", "planar"])
@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("name", ["f16", "bf16"])
def test_compress_golden(mode, bits, name):
    K = _kernels()
    R = torch.from_numpy(GOLDEN[f"R_{mode}"])
    RT = R.T.contiguous()
    rte, rto = RT[:, 0::2].contiguous(), RT[:, 1::2].contiguous()
    b = torch.from_numpy(GOLDEN[f"boundaries_b{bits}"])
    c = torch.from_numpy(GOLDEN[f"centroids_b{bits}"])
    dt = torch.float16 if name == "f16" else torch.bfloat16
    x = torch.from_numpy(GOLDEN[f"x_{name}"].view(np.int16)).view(dt)
    fn = K.planar_compress if mode == "planar" else K.iso_compress
    packed, norms = fn(_dev(x), _dev(rte), _dev(rto), _dev(b))
    key = f"{mode}_b{bits}_{name}"
    assert np.array_equal(packed.cpu().numpy(), GOLDEN[f"packed_{key}"])
    assert np.array_equal(norms.cpu().numpy().view(np.uint32), GOLDEN[f"norms_{key}"].view(np.uint32))
    dec = (K.planar_decompress if mode == "planar" else K.iso_decompress)(packed, norms, _dev(c), dt)
    assert np.array_equal(dec.cpu().view(torch.int16).numpy().view(np.uint16), GOLDEN[f"dec_{key}"])


@pytest.mark.parametrize("n_tokens", [2048, 32768])
@pytest.mark.parametrize("mode,bits", [("iso", 3), ("iso", 4), ("planar", 4)])
def test_compress_config0_full_size(n_tokens, mode, bits):
    """benchmark config 0 (2048 x 8 x 128 fp16, K and V) and a 32768-token run: bit-exact vs oracle."""
    K = _kernels()
    p = Params(mode, bits, bits)
    pn = p.np()
    k, v = kv_config0(n_tokens, 8, 128)
    for x, bnd in ((k, p.kb), (v, p.vb)):
        packed, norms = K.iso_compress(_dev(x), _dev(p.rte), _dev(p.rto), _dev(bnd))
        xb, dt = O.to_bits(x)
        op, on, _, n_ties = O.compress(xb, dt, pn["rte"], pn["rto"], bnd.numpy(), p.blk, want_ties=True)
        gp = packed.cpu().numpy()
        mism = int((gp != op).sum())
        print(f"tokens={n_tokens} {mode}{bits}: mismatched bytes={mism} ties={n_ties}")
        assert mism == 0
        assert np.array_equal(norms.cpu().numpy().view(np.uint32), on.view(np.uint32))
        dec = K.iso_decompress(packed, norms, _dev(p.kc), torch.float16).cpu().float().numpy()
        assert np.array_equal(dec, O.decompress(op, on, p.kc.numpy(), "float16"))


def test_compress_fp32_input():
    K = _kernels()
    p = Params("iso", 3, 3)
    pn = p.np()
    x = torch.randn(64, 8, 128, generator=torch.Generator().manual_seed(7)) * 3
    packed, norms = K.iso_compress(_dev(x), _dev(p.rte), _dev(p.rto), _dev(p.kb))
    op, on = O.compress(x.numpy(), "float32", pn["rte"], pn["rto"], pn["kb"], 4)
    assert np.array_equal(packed.cpu().numpy(), op)
    assert np.array_equal(norms.cpu().numpy().view(np.uint32), on.view(np.uint32))


@pytest.mark.parametrize("H,mode,kb,vb,BS", [(8, "iso", 3, 3, 16), (4, "iso", 4, 3, 16), (8, "planar", 4, 3, 16),
                                             (1, "iso", 3, 4, 16), (2, "planar", 3, 3, 16), (8, "iso", 3, 3, 12),
                                             (4, "iso", 3, 3, 1)])
def test_compress_store_slots_bit_exact(H, mode, kb, vb, BS):
    """Fused K+V compress into random slots: every byte of the cache matches the oracle store
    (block sizes 16, 12 and 1)."""
    K = _kernels()
    p = Params(mode, kb, vb)
    NB = 640 // BS
    N = 300
    k, v = kv_config0(N, H, 128, cfg=3)
    g = torch.Generator().manual_seed(11)
    slots = torch.randperm(NB * BS, generator=g)[:N].to(torch.int64)
    slots[5] = -1  # padding token: skipped
    slots[77] = -1
    cache_ref = np.full((NB, BS, 256 * H), 0xAB, np.uint8)  # sentinel: untouched slots keep it
    pn = p.np()
    kp, kn = O.compress(O.to_bits(k)[0], "float16", pn["rte"], pn["rto"], pn["kb"], p.blk)
    vp, vn = O.compress(O.to_bits(v)[0], "float16", pn["rte"], pn["rto"], pn["vb"], p.blk)
    O.compress_store(cache_ref, slots.numpy(), kp, kn, vp, vn)
    cache = torch.full((NB, BS, 256 * H), 0xAB, dtype=torch.uint8, device="cuda")
    K.compress_store(_dev(k), _dev(v), cache, _dev(slots), _dev(p.rte), _dev(p.rto), _dev(p.kb), _dev(p.vb))
    got = cache.cpu().numpy()
    assert np.array_equal(got, cache_ref), f"{int((got != cache_ref).sum())} bytes differ"


def test_compress_store_strided_qkv_views():
    """key/value as strided views of a fused qkv buffer (vLLM's layout)."""
    K = _kernels()
    p = Params("iso", 3, 3)
    H, HQ, D, N, BS, NB = 8, 32, 128, 50, 16, 8
    qkv = torch.randn(N, (HQ + 2 * H) * D, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    key = qkv[:, HQ * D:(HQ + H) * D].view(N, H, D)
    val = qkv[:, (HQ + H) * D:].view(N, H, D)
    slots = torch.arange(N, dtype=torch.int64)
    cache = torch.zeros(NB, BS, 256 * H, dtype=torch.uint8, device="cuda")
    qkv_d = _dev(qkv)
    K.compress_store(qkv_d[:, HQ * D:(HQ + H) * D].view(N, H, D), qkv_d[:, (HQ + H) * D:].view(N, H, D), cache,
                     _dev(slots), _dev(p.rte), _dev(p.rto), _dev(p.kb), _dev(p.vb))
    ref = build_cache_oracle(key.contiguous(), val.contiguous(), slots.numpy(), NB, BS, p)
    assert np.array_equal(cache.cpu().numpy(), ref)


@pytest.mark.parametrize("H,D", [(8, 128), (3, 80)])
def test_paged_decompress_matches_unique_gather(H, D):
    """Paged decompress == sorted-unique gather + per-row decompress + remap (rq_backend.py:763-852).
    (3, 80): 10 packed dwords per row (a 250-thread expand block) and rows of 3 heads."""
    K = _kernels()
    p = Params("iso", 3, 3) if D == 128 else Params("planar", 3, 3, head_dim=D)
    BS = 16
    lens = [37, 1, 160, 64, 0]
    bt, NB, slots = paged_layout(lens, BS, cfg=4)
    bt[2, 3] = bt[0, 1]  # a block shared by two sequences
    slots_all = np.concatenate(slots)
    total = len(slots_all)
    k, v = kv_config0(total, H, D, cfg=4)
    cache = build_cache_oracle(k, v, slots_all, NB, BS, p)
    kc_ref, vc_ref, bt_ref, U = O.paged_decompress(cache, bt, lens, H, D, p.kc.numpy(), p.vc.numpy(), "bfloat16")
    ok, ov, remap, count = K.paged_decompress(_dev(torch.from_numpy(cache)), _dev(torch.from_numpy(bt)),
                                              _dev(torch.tensor(lens, dtype=torch.int32)), H, D, _dev(p.kc),
                                              _dev(p.vc), torch.bfloat16)
    assert int(count.item()) == U
    assert np.array_equal(remap.cpu().numpy(), bt_ref)
    assert np.array_equal(ok[:U].cpu().float().numpy(), kc_ref)
    assert np.array_equal(ov[:U].cpu().float().numpy(), vc_ref)


def test_cpu_tensors_rejected():
    K = _kernels()
    p = Params()
    with pytest.raises(RuntimeError, match="no CPU path"):
        K.iso_compress(torch.zeros(1, 1, 128, dtype=torch.float16), p.rte, p.rto, p.kb)


def _op_check(x, p, bnd):
    """Op-level compress of x (N, H, D) on the GPU vs the oracle, bit-exact."""
    K = _kernels()
    packed, norms = K.iso_compress(_dev(x), _dev(p.rte), _dev(p.rto), _dev(bnd))
    xb, dt = O.to_bits(x)
    pn = p.np()
    op, on = O.compress(xb, dt, pn["rte"], pn["rto"], bnd.numpy(), p.blk)
    gp = packed.cpu().numpy()
    assert np.array_equal(gp, op), f"{int((gp != op).sum())} packed bytes differ"
    assert np.array_equal(norms.cpu().numpy().view(np.uint32), on.view(np.uint32))


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
def test_compress_extreme_magnitudes(dt):
    """Rows that leave the corrected-division range (norm > 2^40, elements below 2^-60,
    subnormals, all-zero rows) take the plain division and still match bit-exactly."""
    p = Params("iso", 4, 4)
    g = torch.Generator().manual_seed(21)
    x = torch.randn(40, 4, 128, generator=g)
    x[0] = 0.0                                   # all-zero rows
    x[1] *= 1e-30                                # tiny rows (subnormal in bf16/fp32 after scaling)
    x[2] *= 1e-39
    x[3, :, :64] *= 1e-35                        # mixed magnitudes inside a row
    x[4] *= 1e14                                 # norm above 2^40 (fp32/bf16)
    x[5, :, 0] = 3e4                             # one dominant element
    x[6, :, 1::2] = 0.0
    x[7] *= 1e-7                                 # fp16 subnormals
    if dt == torch.float16:
        x[4] = x[8] * 1000                       # keep fp16 finite
    _op_check(x.to(dt), p, p.kb)


@pytest.mark.parametrize("kind", ["duplicate", "close_pair", "uniform", "skewed"])
def test_compress_boundary_sets(kind):
    """Boundary sets that defeat the cell lookup (duplicates, a pair closer than a cell)
    fall back to counting; well-separated but non-Lloyd-Max sets use the lookup."""
    p = Params("iso", 4, 4)
    b = p.kb.clone()
    if kind == "duplicate":
        b[7] = b[6]
    elif kind == "close_pair":
        b[3] = torch.nextafter(b[2], torch.tensor(1.0))
    elif kind == "uniform":
        b = torch.linspace(-0.2, 0.2, 15)
    else:
        b = torch.tensor([-0.3, -0.1, -0.02, 0.0, 0.01, 0.05, 0.2])
    x = torch.randn(96, 8, 128, generator=torch.Generator().manual_seed(3)).to(torch.float16)
    _op_check(x, p, b.float().contiguous())


@pytest.mark.parametrize("D", [64, 80, 256])
@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_compress_head_dims(D, dt):
    p = Params("planar" if D == 80 else "iso", 3, 3, head_dim=D)
    x = torch.randn(33, 3, D, generator=torch.Generator().manual_seed(D)).to(dt)
    _op_check(x, p, p.kb)


@pytest.mark.parametrize("H", [3, 5])
def test_compress_store_heads_not_dividing_workgroup(H):
    """2H rows per token that do not divide a workgroup's 64 rows: tokens straddle
    workgroups, so slot padding and payload come from different workgroups."""
    K = _kernels()
    p = Params("iso", 3, 4)
    BS, NB, N = 16, 20, 200
    k, v = kv_config0(N, H, 128, cfg=4)
    slots = torch.randperm(NB * BS, generator=torch.Generator().manual_seed(H))[:N].to(torch.int64)
    slots[9] = -1
    cache = torch.full((NB, BS, 256 * H), 0xAB, dtype=torch.uint8, device="cuda")
    K.compress_store(_dev(k), _dev(v), cache, _dev(slots), _dev(p.rte), _dev(p.rto), _dev(p.kb), _dev(p.vb))
    ref = np.full((NB, BS, 256 * H), 0xAB, np.uint8)
    pn = p.np()
    kp, kn = O.compress(O.to_bits(k)[0], "float16", pn["rte"], pn["rto"], pn["kb"], p.blk)
    vp, vn = O.compress(O.to_bits(v)[0], "float16", pn["rte"], pn["rto"], pn["vb"], p.blk)
    O.compress_store(ref, slots.numpy(), kp, kn, vp, vn)
    got = cache.cpu().numpy()
    assert np.array_equal(got, ref), f"{int((got != ref).sum())} bytes differ"
