"""GPU parity over seeded random shapes: the fused decode, the int8 prefill and both
non-fused entry points (rq_paged_attention, rq_paged_prefill) against the float64
oracle, on combinations the fixed cases do not enumerate.

Each case draws a kind, kv heads H (1-6 or 8), a GQA group, a block size (1 to 64),
codebooks (iso fast / full or planar, 3 or 4 bits for K and V separately), the query
dtype, K/V scaling and lengths (a third of them at tile and block edges).  The draws
depend only on the case index, so a failing case is reproduced by its id.  Tolerance
as in the other attention tests (rq_testlib.check_tolerance): cos >= 0.999 and
|got - ref| <= max(2e-2, ulp(x) + 2 ulp(rotation-block max)).
"""
import numpy as np
import pytest
import torch

import test_gpu_attention as TA
import test_gpu_decode as TD
import test_gpu_prefill as TP
from rq_testlib import Params, check_tolerance

pytestmark = pytest.mark.gpu

N_CASES = 60
EDGES = [0, 1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129]
_params = {}


def _params_of(mode, kb, vb, iso_mode):
    key = (mode, kb, vb, iso_mode)
    if key not in _params:
        _params[key] = Params(mode, kb, vb, iso_mode=iso_mode) if mode == "iso" else Params(mode, kb, vb)
    return _params[key]


def draw(i):
    """The case of index i: (kind, keyword arguments, description)."""
    rng = np.random.default_rng(9000 + i)
    kind = ["decode", "prefill", "paged_attention", "paged_prefill"][i % 4]
    H = int(rng.choice([1, 2, 3, 4, 5, 6, 8]))
    mode = str(rng.choice(["iso", "planar"]))
    kb, vb = int(rng.choice([3, 4])), int(rng.choice([3, 4]))
    iso_mode = str(rng.choice(["fast", "full"])) if mode == "iso" else "fast"
    dtype = torch.bfloat16 if rng.random() < 0.6 else torch.float16
    BS = int(rng.choice([1, 8, 16, 16, 32, 64]))
    kv = str(rng.choice(["config0", "unit"]))
    if kind == "decode":
        G = int(rng.integers(1, 17))
        B = int(rng.integers(1, 10))
        lens = [int(rng.choice(EDGES)) if rng.random() < 0.3 else int(rng.integers(1, 2500)) for _ in range(B)]
        shape = dict(G=G, lens=lens)
    else:
        G = int(rng.integers(1, 13))
        B = int(rng.integers(1, 5))
        q_lens = [int(x) for x in rng.integers(1, 200, B)]
        ctx = [q + (int(rng.integers(0, 600)) if rng.random() < 0.6 else 0) for q in q_lens]
        shape = dict(G=G, q_lens=q_lens, ctx=ctx)
    desc = (f"{kind} H={H} BS={BS} {mode}{kb}/{vb} {iso_mode if mode == 'iso' else ''} {str(dtype)[6:]} kv={kv} "
            + " ".join(f"{k}={v}" for k, v in shape.items()))
    return kind, dict(H=H, mode=mode, kb=kb, vb=vb, iso_mode=iso_mode, dtype=dtype, BS=BS, kv=kv, **shape), desc


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_shape(i):
    kind, a, desc = draw(i)
    p = _params_of(a["mode"], a["kb"], a["vb"], a["iso_mode"])
    cfg = 200 + i
    H, HQ = a["H"], a["H"] * a["G"]
    if kind == "decode":
        case = TD.decode_case(cfg, len(a["lens"]), H, HQ, a["lens"], block_size=a["BS"], p=p, kv=a["kv"],
                              dtype=a["dtype"])
        got, ref = TD.run_decode(case), TD.ref_decode(case)
    elif kind == "prefill":
        case = TP.prefill_case(cfg, a["q_lens"], a["ctx"], H, HQ, p, kv=a["kv"], BS=a["BS"], dtype=a["dtype"])
        got, ref = TP.run(case), TP.ref(case)
    else:
        case = TA.attn_case(cfg, a["q_lens"], a["ctx"], H, HQ, p, kv=a["kv"], BS=a["BS"], dtype=a["dtype"])
        got, ref = TA.run(case, entry=kind), TA.ref(case)
    err, excess, cs = check_tolerance(got, ref, str(a["dtype"])[6:], 2e-2, 0.999, rot_block=p.blk)
    print(f"{i}: {desc}: max_abs={err:.3e} excess={excess:.3e} cos={cs:.6f}")
    assert np.isfinite(got).all(), desc
    assert excess <= 0 and cs >= 0.999, f"{desc}: max_abs={err} excess={excess} cos={cs}"
