"""GPU parity: int8-MFMA causal prefill vs the float64 oracle.

Tolerance as for decode (rq_testlib.check_tolerance): cos >= 0.999 and
|got - ref| <= max(2e-2, ulp(x_d) + 2 ulp(rotation-block max)); unit-scale
cases also check the plain max-abs <= 2e-2.  Query i of sequence b sits at
position seq_len_b - q_len_b + i.
"""
import numpy as np
import pytest
import torch

import oracle as O
from rq_testlib import Params, build_cache_oracle, check_tolerance, gen, kv_config0, kv_unit, paged_layout

pytestmark = pytest.mark.gpu


def prefill_case(cfg, q_lens, ctx_lens, H, HQ, p, kv="config0", BS=16, dtype=torch.bfloat16):
    bt, NB, slots = paged_layout(ctx_lens, BS, cfg)
    total = int(sum(ctx_lens))
    k, v = (kv_config0(total, H, 128, cfg) if kv == "config0" else kv_unit(total, H, 128, cfg))
    cache = build_cache_oracle(k, v, np.concatenate(slots), NB, BS, p)
    T = int(sum(q_lens))
    q = torch.randn(T, HQ, 128, generator=gen(1000 * cfg + 6)).to(dtype)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    return dict(cache=cache, bt=bt, lens=np.asarray(ctx_lens, np.int32), q=q, cu=cu, H=H, HQ=HQ, BS=BS, p=p,
                q_lens=list(q_lens))


def run(case, use_cu=True):
    from rotorquant_vllm import kernels as K
    p = case["p"]
    d = lambda x: torch.from_numpy(x).to("cuda") if isinstance(x, np.ndarray) else x.to("cuda")  # noqa: E731
    kw = dict(cu_seqlens_q=d(case["cu"]), max_q_len=max(case["q_lens"])) if use_cu else {}
    out = K.fused_paged_rq_int8_prefill(d(case["q"]), d(case["cache"]), d(case["bt"]), d(case["lens"]), d(p.kc),
                                        d(p.vc), d(p.R), case["H"], 128, case["BS"], **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def ref(case):
    p = case["p"]
    dt = str(case["q"].dtype).replace("torch.", "")
    return O.prefill_attention(case["q"].float().numpy(), case["cu"], case["cache"], case["bt"], case["lens"],
                               case["H"], 128, p.kc.numpy(), p.vc.numpy(), p.R.numpy(), 1 / np.sqrt(128), dt)


def check(case, tag, use_cu=True, plain_max_abs=False):
    got, exp = run(case, use_cu), ref(case)
    dt = str(case["q"].dtype).replace("torch.", "")
    err, excess, cs = check_tolerance(got, exp, dt, rot_block=case["p"].blk)
    print(f"{tag}: max_abs={err:.3e} excess_over_bound={excess:.3e} cos={cs:.6f}")
    assert np.isfinite(got).all()
    assert excess <= 0 and cs >= 0.999, f"{tag}: max_abs={err} excess={excess} cos={cs}"
    if plain_max_abs:
        assert err <= 2e-2, f"{tag}: max_abs={err}"


def test_prefill_single_sequence_reference_api():
    """Config 3 layout (32 q / 8 kv, iso fast 4-bit), one fresh sequence, the reference's call form."""
    p = Params("iso", 4, 4)
    case = prefill_case(31, [700], [700], 8, 32, p)
    check(case, "single", use_cu=False)


def test_prefill_varlen_batch_iso4():
    """Several fresh sequences in one launch, ragged lengths around tile edges."""
    p = Params("iso", 4, 4)
    lens = [1, 15, 16, 17, 63, 64, 65, 300]
    check(prefill_case(32, lens, lens, 8, 32, p), "varlen")


def test_prefill_chunked_with_prefix_gqa7():
    """Config 4 style: GQA 7 (28 q / 4 kv), iso full 3-bit, chunks after a cached prefix."""
    p = Params("iso", 3, 3, iso_mode="full")
    case = prefill_case(33, [128, 200], [128 + 500, 200 + 37], 4, 28, p)
    check(case, "chunked-gqa7")


def test_prefill_unit_scale_fp16_planar():
    p = Params("planar", 4, 3)
    case = prefill_case(34, [256, 100], [256, 100], 8, 32, p, kv="unit", dtype=torch.float16)
    check(case, "unit-planar-f16", plain_max_abs=True)


def test_prefill_unit_scale_bf16_iso4():
    """Config 3 codebooks with unit-scale K/V: the plain max-abs <= 2e-2 bound holds."""
    p = Params("iso", 4, 4)
    case = prefill_case(35, [512], [512], 8, 32, p, kv="unit")
    check(case, "unit-iso4-bf16", plain_max_abs=True)


@pytest.mark.parametrize("BS", [12, 32, 64])
def test_prefill_block_sizes(BS):
    """Block sizes other than 16 (a non-power of two among them), chunks after prefixes."""
    p = Params("iso", 4, 4)
    check(prefill_case(36, [70, 1, 130], [70 + 45, 80, 130], 8, 32, p, BS=BS), f"bs{BS}")


def test_prefill_gqa16_one_kv_head():
    """16 query heads on one kv head: the widest workgroup (16 waves), where the per-wave
    output staging buffers fill the tile area; it also takes the plain work order (13
    query blocks do not cut into the 8 XCD slices of a single kv head, and two
    (sequence, kv head) pairs do not divide into the 8 XCDs)."""
    p = Params("iso", 4, 3)
    check(prefill_case(9, [200, 77], [260, 77], 1, 16, p), "gqa16")


@pytest.mark.parametrize("H,HQ,q_lens,ctx_lens", [
    (4, 12, [256, 33, 100], [256 + 300, 33, 100 + 1000]),  # GQA 3: 6 workgroups per pair, 2 XCD slices
    (2, 10, [512, 300], [512 + 200, 300]),                 # GQA 5: 20 workgroups per pair, 4 XCD slices
    (2, 12, [96, 40], [96 + 64, 40 + 513]),                # GQA 6: 36 units in 5 workgroups, plain order
])
def test_prefill_gqa_flattened_workgroups(H, HQ, q_lens, ctx_lens):
    """GQA groups of 3, 5 and 6 query heads: 8-wave workgroups over the sequence's
    (16-position group, query head) units in position-group-major order, so a
    workgroup's waves span two position groups (different causal limits) and the last
    workgroup of a sequence has waves with no unit; ragged query lengths, chunks after
    prefixes, with and without the XCD slices of the work order."""
    p = Params("iso", 3, 3, iso_mode="full")
    check(prefill_case(37 + HQ // H, q_lens, ctx_lens, H, HQ, p), f"gqa{HQ // H}-flat H={H}")


def test_prefill_multi_sequence_requires_cu_seqlens():
    from rotorquant_vllm import kernels as K
    p = Params()
    with pytest.raises(ValueError, match="single sequence"):
        K.fused_paged_rq_int8_prefill(torch.zeros(4, 32, 128, dtype=torch.bfloat16, device="cuda"),
                                      torch.zeros(2, 16, 2048, dtype=torch.uint8, device="cuda"),
                                      torch.zeros(2, 1, dtype=torch.int32, device="cuda"),
                                      torch.tensor([2, 2], dtype=torch.int32, device="cuda"), p.kc.cuda(),
                                      p.vc.cuda(), p.R.cuda(), 8, 128, 16)
