"""GPU parity: fused paged decode vs the float64 oracle.

Tolerance (rq_testlib.check_tolerance): cos >= 0.999 and |got - ref| <=
max(2e-2, ulp(x_d) + 2 ulp(rotation-block max)) elementwise (the reference
rounds twice, see there); unit-scale cases check the plain max-abs <= 2e-2.

The oracle dequantizes the same packed cache bit-exactly and runs exact
softmax attention in the rotated space with the query rounded like the
reference's q_rot, then rotates back (fused_paged_rq_decode.py:271, :308).
"""
import numpy as np
import pytest
import torch

import oracle as O
from rq_testlib import Params, check_tolerance, decode_case, identical_keys_case, lens_loguniform, lens_uniform

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MIN_COS = 0.999


def run_decode(case):
    from rotorquant_vllm import kernels as K
    p = case["p"]
    q = case["q"].to("cuda")
    out = K.fused_paged_rq_decode(q, torch.from_numpy(case["cache"]).to("cuda"), torch.from_numpy(case["bt"]).to("cuda"),
                                  torch.from_numpy(case["lens"]).to("cuda"), p.kc.to("cuda"), p.vc.to("cuda"),
                                  p.R.to("cuda"), case["H"], p.D, case["BS"], sm_scale=case["sm_scale"])
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def ref_decode(case):
    p = case["p"]
    dt = str(case["q"].dtype).replace("torch.", "")
    return O.decode_attention(case["q"].float().numpy(), case["cache"], case["bt"], case["lens"], case["H"], p.D,
                              p.kc.numpy(), p.vc.numpy(), p.R.numpy(), case["sm_scale"], dt)


def check(case, tag, plain_max_abs=False):
    got = run_decode(case)
    ref = ref_decode(case)
    dt = str(case["q"].dtype).replace("torch.", "")
    err, excess, cs = check_tolerance(got, ref, dt, MAX_ABS, MIN_COS, rot_block=case["p"].blk)
    print(f"{tag}: max_abs={err:.3e} excess_over_bound={excess:.3e} cos={cs:.6f}")
    assert np.isfinite(got).all()
    assert excess <= 0 and cs >= MIN_COS, f"{tag}: max_abs={err} excess={excess} cos={cs}"
    if plain_max_abs:
        assert err <= MAX_ABS, f"{tag}: max_abs={err}"
    return got, ref


def test_decode_unit_scale_plain_tolerance():
    """K, V ~ N(0,1): outputs within a few units, so the plain bound max-abs <= 2e-2 applies."""
    lens = lens_uniform(8, 1024, 8192, cfg=8)
    check(decode_case(8, 8, 8, 32, lens, kv="unit"), "unit-scale", plain_max_abs=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_config1_shape_small_batch(dtype):
    """Llama-3-8B layer shape (32 q / 8 kv, D 128), iso fast 3-bit, 8 sequences of 1024..8192."""
    lens = lens_uniform(8, 1024, 8192, cfg=1)
    check(decode_case(1, 8, 8, 32, lens, dtype=dtype), f"cfg1-small {dtype}")


def test_decode_many_short_sequences():
    """112 sequences x 32 query heads (more merge waves than fit at once at the wide
    merge's occupancy): the merge runs its 16-segment variant."""
    lens = lens_uniform(112, 1, 300, cfg=12)
    check(decode_case(12, len(lens), 8, 32, lens), "many-short")


def test_decode_ragged_edges():
    """Lengths 0, 1, 15, 16, 17, 31, 33, 255, 256, 257, 1000 (tile / block / chunk edges)."""
    lens = [0, 1, 15, 16, 17, 31, 33, 255, 256, 257, 1000]
    check(decode_case(11, len(lens), 8, 32, lens), "ragged")


def test_decode_planar_asym_k4_v3():
    """Config 2 head layout and codebooks: planar K 4-bit / V 3-bit, keys with 10x outlier channels."""
    p = Params("planar", 4, 3)
    lens = lens_loguniform(6, 2048, 32768, cfg=2)
    check(decode_case(2, 6, 8, 32, lens, p=p, kv="outlier"), "cfg2-planar")


def test_decode_gqa7_iso_full():
    """Config 4 head layout: 28 q / 4 kv heads (GQA 7), iso full 3-bit, one long context."""
    p = Params("iso", 3, 3, iso_mode="full")
    lens = [20000, 512, 3000, 16384]
    check(decode_case(4, 4, 4, 28, lens, p=p), "cfg4-gqa7")


@pytest.mark.parametrize("H,HQ", [(1, 4), (2, 8)])
def test_decode_tensor_parallel_slices(H, HQ):
    """One GPU's share of the config-1 layer under tensor parallelism (TP 8: 1 kv / 4 q
    heads; TP 4: 2 / 8): one or two waves per decode workgroup."""
    lens = lens_uniform(8, 1024, 8192, cfg=14)
    check(decode_case(14, 8, H, HQ, lens), f"tp-slice H={H} HQ={HQ}")


def test_decode_tp8_slice_many_sequences():
    """The TP-8 slice's head layout (1 kv / 4 q heads) with 64 short sequences: each
    sequence spans ~32 one-wave decode workgroups, and the merge gives each (sequence,
    query head) four waves that take every fourth 16-segment pass (most of them with
    empty ranges here: 64 sequences of 1..400 tokens hold far fewer tiles than there
    are workgroups)."""
    lens = lens_uniform(64, 1, 400, cfg=23)
    check(decode_case(23, len(lens), 1, 4, lens), "tp8-many")


@pytest.mark.parametrize("H,HQ,lens", [(2, 8, [60000, 3000, 1]), (1, 4, [40000])])
def test_decode_long_context_few_sequences(H, HQ, lens):
    """A long context in a small batch: the sequence spans ~1000 two-wave or ~2000
    one-wave decode workgroups, so each of the four merge waves of a (sequence, head)
    pair runs several 32-segment passes before their states are combined."""
    check(decode_case(24 + H, len(lens), H, HQ, lens), f"long-few H={H} lens={lens}")


@pytest.mark.parametrize("H,HQ,dtype", [(2, 32, torch.bfloat16), (1, 12, torch.bfloat16), (4, 40, torch.float16),
                                         (3, 12, torch.bfloat16), (6, 12, torch.float16), (5, 40, torch.bfloat16)])
def test_decode_head_layouts(H, HQ, dtype):
    """Head layouts beyond the benchmark ones: GQA groups above 8 (two MFMAs per pair of
    head dims; 16, 12 and 10 query heads per kv head) with one, two and four kv heads per
    workgroup, and kv-head counts without a power-of-two divisor up to 8 (3, 6, 5 waves per
    workgroup: the variant with the head count taken at run time)."""
    lens = [1, 31, 33, 700, 2500]
    check(decode_case(16 + H, len(lens), H, HQ, lens, dtype=dtype), f"heads H={H} HQ={HQ} {dtype}")


@pytest.mark.parametrize("BS", [1, 12, 64, 128])
def test_decode_block_sizes(BS):
    """Block sizes other than 16: one token per block, a non-power of two (division
    instead of shifts), and blocks larger than a 32-token tile."""
    lens = [1, 70, 300, 1000]
    check(decode_case(15, len(lens), 8, 32, lens, block_size=BS), f"bs{BS}")


@pytest.mark.parametrize("mode", ["iso", "planar"])
def test_decode_4bit_kv_config1_heads(mode):
    """RQ_BITS=4 on the config-1 head layout (32 q / 8 kv heads): 4-bit V takes
    workgroups of four kv heads (two per kv-head set), with 16-entry K and V tables."""
    lens = [1, 33, 700, 2500, 8000, 4096]
    check(decode_case(21, len(lens), 8, 32, lens, p=Params(mode, 4, 4)), f"4bit {mode}")


def test_decode_k3_v4_and_block_size_32():
    p = Params("iso", 3, 4)
    lens = [700, 33, 64]
    check(decode_case(5, 3, 8, 16, lens, block_size=32, p=p), "k3v4-bs32")


def test_decode_closed_forms():
    """Closed forms, no attention oracle: L = 1 -> the R-rotated V row; identical keys
    (every cached key the same vector) -> the R-rotated mean of V, at 8 kv heads x GQA 4
    and at GQA 7 over 2000 tokens (many tiles, several decode workgroups)."""
    case = decode_case(6, 2, 8, 32, [1, 1])
    got = run_decode(case)
    p = case["p"]
    dt = "bfloat16"
    for b in range(2):
        K, V = O.gather_seq(case["cache"], case["bt"][b], 1, 8, 128, p.kc.numpy(), p.vc.numpy())
        for h in range(32):
            exp = O.unrotate_out(V[0, h // 4][None, :], p.R.numpy(), dt)[0]
            _, excess, cs = check_tolerance(got[b, h], exp, dt, 1e-2, rot_block=p.blk)
            assert excess <= 0 and cs >= 0.9999
    for L, H, HQ, mode in ((333, 8, 32, "fast"), (2000, 4, 28, "full")):
        case = identical_keys_case(cfg=45, L=L, H=H, HQ=HQ, p=Params("iso", 3, 3, iso_mode=mode))
        got = run_decode(case)
        p = case["p"]
        K, V = O.gather_seq(case["cache"], case["bt"][0], L, H, 128, p.kc.numpy(), p.vc.numpy())
        assert np.all(K == K[0:1]), "the case must hold identical keys"
        mean = V.mean(axis=0)  # (H, D), float64
        G = HQ // H
        exp = O.unrotate_out(np.stack([mean[h // G] for h in range(HQ)]), p.R.numpy(), dt)
        err, excess, cs = check_tolerance(got[0], exp, dt, rot_block=p.blk)
        print(f"identical keys L={L} H={H} HQ={HQ}: max_abs={err:.3e} excess={excess:.3e} cos={cs:.6f}")
        assert excess <= 0 and cs >= 0.9999


def test_decode_deterministic_and_batch_consistent():
    """The same batch decoded twice gives identical bits.  A sequence decoded alone
    and inside a batch of long sequences agrees within the parity tolerance (work
    is split evenly over the whole batch, so the split points -- and the fp32
    summation order -- depend on the batch)."""
    lens = [5000, 6000, 7000]
    case = decode_case(7, 3, 8, 32, lens)
    got_all = run_decode(case)
    assert np.array_equal(got_all, run_decode(case))
    one = dict(case)
    one["bt"] = case["bt"][1:2]
    one["lens"] = case["lens"][1:2]
    one["q"] = case["q"][1:2]
    got_one = run_decode(one)
    _, excess, cs = check_tolerance(got_one[0], got_all[1], "bfloat16", MAX_ABS, MIN_COS, rot_block=case["p"].blk)
    assert excess <= 0 and cs >= 0.9999


def test_decode_timed_entry_point():
    """rq_fused_decode_timed gives rq_fused_decode's output bit for bit and records
    its events around the decode kernel: a positive time, shorter than the whole
    call timed by events on the stream around it."""
    from rotorquant_vllm import kernels as K
    lens = [3000, 700, 5000, 64]
    case = decode_case(22, 4, 8, 32, lens)
    p = case["p"]
    dev = torch.device("cuda")
    args = (case["q"].to(dev), torch.from_numpy(case["cache"]).to(dev), torch.from_numpy(case["bt"]).to(dev),
            torch.from_numpy(case["lens"]).to(dev), p.kc.to(dev), p.vc.to(dev), p.R.to(dev), 8, 128, 16)
    plain = K.fused_paged_rq_decode_launcher(*args, sm_scale=case["sm_scale"])
    ref = plain().clone()
    k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    timed = K.fused_paged_rq_decode_launcher(*args, sm_scale=case["sm_scale"], kernel_events=(k0, k1))
    torch.cuda.synchronize()
    for _ in range(3):
        c0.record()
        got = timed()
        c1.record()
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        t_kernel, t_call = k0.elapsed_time(k1), c0.elapsed_time(c1)
        print(f"decode kernel {t_kernel * 1e3:.1f} us, call {t_call * 1e3:.1f} us")
        assert 0 < t_kernel < t_call


def test_decode_graph_replay_matches_eager():
    """rq_fused_decode captured in a HIP graph: each of several replays, with eager
    calls on other inputs in between, reproduces the eager result bit for bit."""
    from rotorquant_vllm import _lib
    from rotorquant_vllm import kernels as K
    lens = [700, 4000, 33, 2500]
    case = decode_case(9, 4, 8, 32, lens)
    other = decode_case(10, 2, 8, 32, [300, 5000])
    p = case["p"]
    dev = torch.device("cuda")
    args = dict(num_kv_heads=8, head_dim=128, block_size=16, sm_scale=case["sm_scale"])
    cache, bt, sl = (torch.from_numpy(case[k]).to(dev) for k in ("cache", "bt", "lens"))
    ocache, obt, osl = (torch.from_numpy(other[k]).to(dev) for k in ("cache", "bt", "lens"))
    q, oq = case["q"].to(dev), other["q"].to(dev)
    kc, vc, R = p.kc.to(dev), p.vc.to(dev), p.R.to(dev)
    need = _lib.load().rq_fused_decode_workspace_bytes(4, 32, 128, max(lens))
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    out = torch.empty_like(q)

    def call():
        K.fused_paged_rq_decode(q, cache, bt, sl, kc, vc, R, out=out, max_seq_len=max(lens), workspace=ws, **args)

    call()
    torch.cuda.synchronize()
    eager = out.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for _ in range(3):
        out.zero_()
        K.fused_paged_rq_decode(oq, ocache, obt, osl, kc, vc, R, max_seq_len=5000, **args)  # eager work between
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
