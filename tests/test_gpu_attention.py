"""GPU parity: the non-fused path's kernels vs the float64 oracle -- rq_paged_attention
(one kernel, K/V tiles dequantized in LDS) and rq_paged_prefill (each 64-key tile
decoded once into a workspace, then attention), every case run through both.

The oracle is oracle.unfused_attention: the reference's non-fused path
(rq_backend.py:937-1036) with K/V decompressed to the q dtype and the
attention computed exactly.  Tolerance as for the fused kernels
(rq_testlib.check_tolerance): cos >= 0.999 and |got - ref| <= max(2e-2,
ulp(x) + 2 ulp(rotation-block max)); unit-scale cases also check the plain
max-abs <= 2e-2.  Query i of sequence b sits at position seq_len_b - q_len_b + i.
"""
import numpy as np
import pytest
import torch

import oracle as O
from rq_testlib import Params, build_cache_oracle, check_tolerance, gen, kv_config0, kv_unit, paged_layout

pytestmark = pytest.mark.gpu


def attn_case(cfg, q_lens, ctx_lens, H, HQ, p, kv="config0", BS=16, dtype=torch.bfloat16):
    bt, NB, slots = paged_layout(ctx_lens, BS, cfg)
    total = int(sum(ctx_lens))
    k, v = (kv_config0(total, H, 128, cfg) if kv == "config0" else kv_unit(total, H, 128, cfg))
    cache = build_cache_oracle(k, v, np.concatenate(slots), NB, BS, p)
    q = torch.randn(int(sum(q_lens)), HQ, 128, generator=gen(1000 * cfg + 7)).to(dtype)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    return dict(cache=cache, bt=bt, lens=np.asarray(ctx_lens, np.int32), q=q, cu=cu, H=H, HQ=HQ, BS=BS, p=p,
                q_lens=list(q_lens))


def _dev(x):
    return torch.from_numpy(x).to("cuda") if isinstance(x, np.ndarray) else x.to("cuda")


ENTRIES = ["paged_attention", "paged_prefill"]


@pytest.fixture(params=ENTRIES)
def entry(request):
    return request.param


def run(case, causal=True, out=None, entry="paged_attention"):
    from rotorquant_vllm import kernels as K
    p = case["p"]
    res = getattr(K, entry)(_dev(case["q"]), _dev(case["cache"]), _dev(case["bt"]), _dev(case["lens"]),
                            _dev(case["cu"]), max(case["q_lens"]), _dev(p.kc), _dev(p.vc), _dev(p.R), case["H"], 128,
                            case["BS"], causal=causal, out=out)
    torch.cuda.synchronize()
    return res.float().cpu().numpy()


def ref(case, causal=True):
    p = case["p"]
    dt = str(case["q"].dtype).replace("torch.", "")
    return O.unfused_attention(case["q"].float().numpy(), case["cu"], case["cache"], case["bt"], case["lens"],
                               case["H"], 128, p.kc.numpy(), p.vc.numpy(), p.R.numpy(), 1 / np.sqrt(128), dt,
                               causal=causal)


def check(case, tag, causal=True, plain_max_abs=False, entry="paged_attention"):
    tag = f"{entry}/{tag}"
    print(f"{tag}: seqs={len(case['q_lens'])} q={case['q_lens'][:8]} ctx={case['lens'].tolist()[:8]} "
          f"H={case['H']} HQ={case['HQ']} BS={case['BS']} causal={causal}", flush=True)
    got, exp = run(case, causal, entry=entry), ref(case, causal)
    dt = str(case["q"].dtype).replace("torch.", "")
    err, excess, cs = check_tolerance(got, exp, dt, rot_block=case["p"].blk)
    print(f"{tag}: max_abs={err:.3e} excess_over_bound={excess:.3e} cos={cs:.7f}", flush=True)
    assert np.isfinite(got).all()
    assert excess <= 0 and cs >= 0.999, f"{tag}: max_abs={err} excess={excess} cos={cs}"
    if plain_max_abs:
        assert err <= 2e-2, f"{tag}: max_abs={err}"


def test_attention_chunks_after_prefixes_iso3(entry):
    """Config 1 heads (32 q / 8 kv), iso fast 3-bit; ragged chunks around tile edges after prefixes."""
    q_lens = [1, 15, 16, 17, 64, 65, 130]
    ctx = [q + pre for q, pre in zip(q_lens, [0, 40, 64, 100, 0, 191, 300])]
    check(attn_case(61, q_lens, ctx, 8, 32, Params("iso", 3, 3)), "chunks-iso3", entry=entry)


def test_attention_decode_batch_one_token_each(entry):
    """max_q_len = 1: one 16-position group per workgroup; contexts around tile edges and long."""
    ctx = [1, 2, 63, 64, 65, 129, 1000, 3001]
    check(attn_case(62, [1] * len(ctx), ctx, 8, 32, Params("iso", 3, 3)), "decode-batch", entry=entry)


def test_attention_gqa7_iso_full_mixed(entry):
    """Config 4 heads (28 q / 4 kv, GQA 7), iso full 3-bit; decodes and chunks in one launch."""
    q_lens = [1, 1, 200, 64]
    ctx = [500, 77, 200 + 350, 64 + 1]
    check(attn_case(63, q_lens, ctx, 4, 28, Params("iso", 3, 3, iso_mode="full")), "gqa7-mixed", entry=entry)


@pytest.mark.parametrize("H,HQ", [(2, 32), (2, 24), (1, 9), (8, 8), (4, 12)])
def test_attention_gqa_widths(H, HQ, entry):
    """GQA 16 / 12 / 9 split over 2 / 2 / 3 workgroups per kv head; GQA 1 and 3 take 4+ waves."""
    q_lens = [33, 1, 100]
    ctx = [33 + 20, 90, 100]
    check(attn_case(64 + HQ, q_lens, ctx, H, HQ, Params("planar", 4, 3)), f"gqa{HQ // H}", entry=entry)


def test_attention_noncausal(entry):
    """causal = 0: every query of a sequence sees all its keys."""
    q_lens = [50, 1, 70]
    ctx = [50 + 13, 40, 70]
    check(attn_case(65, q_lens, ctx, 8, 32, Params("iso", 4, 4)), "noncausal", causal=False, entry=entry)


def test_attention_unit_scale_fp16_planar(entry):
    """Unit-scale K/V and fp16 q: the plain 2e-2 bound holds too."""
    q_lens = [80, 1, 40]
    ctx = [80 + 64, 300, 40]
    check(attn_case(66, q_lens, ctx, 8, 32, Params("planar", 3, 3), kv="unit", dtype=torch.float16), "unit-fp16",
          plain_max_abs=True, entry=entry)


@pytest.mark.parametrize("BS", [12, 32])
def test_attention_block_sizes(BS, entry):
    """Block size 12 (no power of two) and 32."""
    q_lens = [20, 1, 45]
    ctx = [20 + 31, 100, 45]
    check(attn_case(67, q_lens, ctx, 8, 32, Params("iso", 3, 3), BS=BS), f"bs{BS}", entry=entry)


def test_attention_empty_sequences(entry):
    """Sequences without query tokens, with or without context, between ones that have
    them: their work items exit at once, and the other sequences' rows are unaffected."""
    q_lens = [0, 20, 0, 33, 0]
    ctx = [0, 25, 7, 33, 0]
    check(attn_case(72, q_lens, ctx, 8, 32, Params("iso", 3, 3)), "empty-seqs", entry=entry)


def test_attention_single_key_closed_form(entry):
    """L = 1: the output is the back-rotated V row (rounded to bf16 twice), bit-exact
    up to the oracle's rounding of the same value."""
    case = attn_case(68, [1, 1], [1, 1], 2, 8, Params("iso", 4, 4))
    got, exp = run(case, entry=entry), ref(case)
    assert np.abs(got - exp).max() <= 1e-2 * max(1.0, float(np.abs(exp).max()))


def test_attention_graph_replay():
    """The call captured in a HIP graph: each replay, after the eager work between
    replays (new q and context lengths written into the captured buffers), equals
    the eager call on the same inputs."""
    from rotorquant_vllm import kernels as K
    q_lens = [1, 1, 1, 1]
    ctx = [300, 65, 64, 1000]
    case = attn_case(69, q_lens, ctx, 8, 32, Params("iso", 3, 3))
    p = case["p"]
    q, cache, bt = _dev(case["q"]), _dev(case["cache"]), _dev(case["bt"])
    lens, cu = _dev(case["lens"]), _dev(case["cu"])
    kc, vc, R = _dev(p.kc), _dev(p.vc), _dev(p.R)
    out = torch.empty_like(q)
    args = (q, cache, bt, lens, cu, 1, kc, vc, R, 8, 128, 16)
    K.paged_attention(*args, out=out)  # warm-up (rotation block, library load)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            K.paged_attention(*args, out=out)
    torch.cuda.synchronize()
    for r in range(3):
        q.copy_(torch.randn(q.shape, generator=gen(700 + r)).to(q.dtype).to("cuda"))
        lens.copy_(torch.tensor([300 - 50 * r, 65 + r, 64, 1000 - 7 * r], dtype=torch.int32))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = K.paged_attention(*args)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), f"replay {r}"


@pytest.mark.parametrize("causal", [True, False])
def test_paged_prefill_equals_paged_attention(causal):
    """Same arithmetic in both kernels (K/V rounded to the q dtype, the same fp32
    online softmax over the same 64-key tiles): outputs equal bit for bit on a
    mixed batch -- decodes, a chunk after a long prefix, ragged tails -- and also
    through a view of a larger output tensor (strided rows)."""
    q_lens = [1, 3, 17, 64, 129, 700]
    ctx = [900, 5, 17 + 333, 64, 129 + 1, 700 + 64]
    case = attn_case(71, q_lens, ctx, 8, 32, Params("iso", 3, 3))
    a = run(case, causal, entry="paged_attention")
    b = run(case, causal, entry="paged_prefill")
    assert np.array_equal(a, b)
    big = torch.zeros(case["q"].shape[0], 40, 128, dtype=case["q"].dtype, device="cuda")
    c = run(case, causal, out=big[:, 4:36], entry="paged_prefill")
    assert np.array_equal(a, c)
    assert torch.all(big[:, :4] == 0) and torch.all(big[:, 36:] == 0)
