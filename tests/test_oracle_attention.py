"""Pins of the oracle's attention (CPU): decode_attention / prefill_attention.

The GPU parity tests judge the kernels against oracle.decode_attention and
oracle.prefill_attention; this file pins those two functions themselves,
without the kernels, against:

  * torch.nn.functional.scaled_dot_product_attention in float64, over K/V
    dequantized here with torch ops from the cache bytes (block-table walk,
    nibble split, centroid * norm in fp32) and cast by torch to the q dtype as
    both reference kernels cast them (fused_paged_rq_decode.py:146-147,
    :190-191; fused_paged_rq_int8_prefill.py:172, :224), GQA by
    repeat_interleave and an explicit causal mask at positions L - T + i;
  * closed forms: zero context -> zeros, L = 1 -> the V row, identical keys ->
    the mean of V, two keys -> the logistic weight of sm_scale * (s1 - s0);
  * consistency: prefill row i of a chunk equals decode over the first
    L - T + i + 1 keys (T = L and T < L);
  * the q / output roundings against torch's own fp32 matmul and casts
    (fused_paged_rq_decode.py:271, :201-206, :308).

Planted mistakes (GQA map h % H instead of h // G, the causal mask one
position off either way, the score scale dropped, K/V left as unrounded fp32
products) go into the oracle through its helpers _kv_head / _visible /
_scores / decompress, and each must fail a check here.

Reference kernel math: src/rotorquant_vllm/triton/fused_paged_rq_decode.py:76-206,
fused_paged_rq_int8_prefill.py:187-189.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from rq_testlib import Params, build_cache_oracle, decode_case, gen, identical_keys_case, kv_config0, paged_layout

D = 128


# ---------------------------------------------------------------------------
# Independent pieces (torch)
# ---------------------------------------------------------------------------

def torch_dequant(cache: np.ndarray, bt_row, L: int, H: int, kc, vc, cast=None):
    """K, V (L, H, D) float64 from the cache bytes, with torch ops only; with cast
    (a torch dtype), the fp32 products are cast to it as the reference kernels do.

    Slot layout: [K idx H x 64 | K norms H x f32 | V idx | V norms | pad];
    byte j of a head holds dim 2j in its high nibble and dim 2j + 1 in its low one."""
    c = torch.from_numpy(cache)
    BS = c.shape[1]
    pos = torch.arange(L)
    phys = torch.as_tensor(np.asarray(bt_row), dtype=torch.long)[pos // BS]
    slot = c[phys, pos % BS]  # (L, TB) uint8
    half = D // 2

    def part(idx_off, norm_off, cb):
        b = slot[:, idx_off:idx_off + H * half].reshape(L, H, half).long()
        idx = torch.stack([b >> 4, b & 15], dim=-1).reshape(L, H, D)
        nrm = slot[:, norm_off:norm_off + 4 * H].contiguous().view(torch.float32).reshape(L, H, 1)
        vals = torch.as_tensor(np.asarray(cb), dtype=torch.float32)[idx] * nrm  # one fp32 product
        return (vals if cast is None else vals.to(cast)).double()

    K = part(0, H * half, kc)
    V = part(H * half + 4 * H, 2 * H * half + 4 * H, vc)
    return K, V


def torch_q_rot(q: torch.Tensor, R: torch.Tensor, dtype=torch.bfloat16) -> torch.Tensor:
    """(q.float() @ R^T).to(dtype): the reference's pre-rotation (fused_paged_rq_decode.py:271)."""
    return (q.float() @ R.T.float()).to(dtype).double()


def sdpa_rot(q_rot: torch.Tensor, K: torch.Tensor, V: torch.Tensor, G: int, pos_q, sm_scale: float) -> torch.Tensor:
    """float64 SDPA: q_rot (T, HQ, D), K/V (L, H, D); query t sees keys <= pos_q[t]."""
    L = K.shape[0]
    k = K.transpose(0, 1).repeat_interleave(G, dim=0)[None]  # (1, HQ, L, D)
    v = V.transpose(0, 1).repeat_interleave(G, dim=0)[None]
    mask = torch.arange(L)[None, :] <= torch.as_tensor(pos_q)[:, None]
    o = F.scaled_dot_product_attention(q_rot.transpose(0, 1)[None], k, v, attn_mask=mask, scale=sm_scale)
    return o[0].transpose(0, 1)  # (T, HQ, D)


def rel_err(a, b) -> float:
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


# ---------------------------------------------------------------------------
# Cases and checks (each returns an error; tests assert it small, mutants large)
# ---------------------------------------------------------------------------

def _decode_case():
    p = Params("iso", 3, 3, iso_mode="full")
    return decode_case(41, 4, 2, 8, [0, 37, 300, 1000], p=p)


def check_decode_vs_sdpa(case) -> float:
    p = case["p"]
    pn = p.np()
    dt = "bfloat16"
    got = O.decode_attention_rot(case["q"].float().numpy(), case["cache"], case["bt"], case["lens"], case["H"], D,
                                 pn["kc"], pn["vc"], pn["R"], case["sm_scale"], dt)
    err = 0.0
    G = case["HQ"] // case["H"]
    for b, L in enumerate(case["lens"]):
        L = int(L)
        if L == 0:
            err = max(err, float(np.abs(got[b]).max()))
            continue
        K, V = torch_dequant(case["cache"], case["bt"][b], L, case["H"], pn["kc"], pn["vc"], cast=torch.bfloat16)
        qr = torch_q_rot(case["q"][b:b + 1], p.R)
        exp = sdpa_rot(qr, K, V, G, [L - 1], case["sm_scale"])[0].numpy()
        err = max(err, rel_err(got[b], exp))
    return err


def _prefill_case(cfg=42):
    """GQA 7 (28 q / 4 kv heads), chunks after cached prefixes plus one fresh sequence."""
    p = Params("iso", 3, 3, iso_mode="full")
    q_lens, ctx = [40, 70, 33], [40 + 90, 70, 33 + 5]
    bt, NB, slots = paged_layout(ctx, 16, cfg)
    k, v = kv_config0(sum(ctx), 4, D, cfg)
    cache = build_cache_oracle(k, v, np.concatenate(slots), NB, 16, p)
    q = torch.randn(sum(q_lens), 28, D, generator=gen(1000 * cfg + 6)).to(torch.bfloat16)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    return dict(p=p, cache=cache, bt=bt, lens=np.asarray(ctx, np.int32), q=q, cu=cu, H=4, HQ=28,
                sm_scale=1 / math.sqrt(D))


def check_prefill_vs_sdpa(case) -> float:
    p = case["p"]
    pn = p.np()
    got = O.prefill_attention_rot(case["q"].float().numpy(), case["cu"], case["cache"], case["bt"], case["lens"],
                                  case["H"], D, pn["kc"], pn["vc"], pn["R"], case["sm_scale"], "bfloat16")
    err = 0.0
    G = case["HQ"] // case["H"]
    for b in range(len(case["lens"])):
        s0, s1, L = int(case["cu"][b]), int(case["cu"][b + 1]), int(case["lens"][b])
        K, V = torch_dequant(case["cache"], case["bt"][b], L, case["H"], pn["kc"], pn["vc"], cast=torch.bfloat16)
        qr = torch_q_rot(case["q"][s0:s1], p.R)
        T = s1 - s0
        exp = sdpa_rot(qr, K, V, G, [L - T + i for i in range(T)], case["sm_scale"]).numpy()
        err = max(err, rel_err(got[s0:s1], exp))
    return err


def check_prefill_rows_are_prefix_decodes(case) -> float:
    """Row i of sequence b (position L - T + i) equals decode over the first L - T + i + 1 keys."""
    p = case["p"]
    pn = p.np()
    args = (case["H"], D, pn["kc"], pn["vc"], pn["R"], case["sm_scale"], "bfloat16")
    pre = O.prefill_attention_rot(case["q"].float().numpy(), case["cu"], case["cache"], case["bt"], case["lens"],
                                  *args)
    err = 0.0
    for b in range(len(case["lens"])):
        s0, s1, L = int(case["cu"][b]), int(case["cu"][b + 1]), int(case["lens"][b])
        T = s1 - s0
        for i in sorted({0, 1, T // 2, T - 1}):
            dec = O.decode_attention_rot(case["q"][s0 + i:s0 + i + 1].float().numpy(), case["cache"],
                                         case["bt"][b:b + 1], np.asarray([L - T + i + 1]), *args)
            err = max(err, rel_err(pre[s0 + i], dec[0]))
    return err


def check_two_keys(sm_scale=1 / math.sqrt(D)) -> float:
    """L = 2: out = (v0 + e^d v1) / (1 + e^d), d = sm_scale (q.k1 - q.k0)."""
    case = decode_case(43, 1, 1, 2, [2], p=Params("planar", 4, 3))
    p = case["p"]
    pn = p.np()
    got = O.decode_attention_rot(case["q"].float().numpy(), case["cache"], case["bt"], case["lens"], 1, D, pn["kc"],
                                 pn["vc"], pn["R"], sm_scale, "bfloat16")[0]
    K, V = torch_dequant(case["cache"], case["bt"][0], 2, 1, pn["kc"], pn["vc"], cast=torch.bfloat16)
    qr = torch_q_rot(case["q"][0], p.R).numpy()  # (2, D)
    err = 0.0
    for h in range(2):
        s = [float(qr[h] @ K[j, 0].numpy()) for j in range(2)]
        w1 = 1.0 / (1.0 + math.exp(-sm_scale * (s[1] - s[0])))
        exp = (1 - w1) * V[0, 0].numpy() + w1 * V[1, 0].numpy()
        err = max(err, rel_err(got[h], exp))
    return err


# ---------------------------------------------------------------------------
# Tests
# ---------------------------------------------------------------------------

def test_decode_matches_float64_sdpa():
    assert check_decode_vs_sdpa(_decode_case()) < 1e-10


def test_prefill_matches_float64_sdpa_with_prefix_offset():
    assert check_prefill_vs_sdpa(_prefill_case()) < 1e-10


def test_prefill_rows_equal_prefix_decodes():
    """T = L (fresh sequence) and T < L (chunk after a prefix) both covered by the case."""
    assert check_prefill_rows_are_prefix_decodes(_prefill_case()) < 1e-12


def test_two_key_closed_form():
    assert check_two_keys() < 1e-10


def test_zero_context_and_single_key():
    """L = 0 -> zeros; L = 1 -> the dequantized V row (cast to the q dtype) of the query head's kv head."""
    case = decode_case(44, 2, 2, 8, [0, 1])
    pn = case["p"].np()
    got = O.decode_attention_rot(case["q"].float().numpy(), case["cache"], case["bt"], case["lens"], 2, D, pn["kc"],
                                 pn["vc"], pn["R"], case["sm_scale"], "bfloat16")
    assert np.all(got[0] == 0)
    _, V = torch_dequant(case["cache"], case["bt"][1], 1, 2, pn["kc"], pn["vc"], cast=torch.bfloat16)
    for h in range(8):
        assert np.array_equal(got[1, h], V[0, h // 4].numpy())
    full = O.decode_attention(case["q"].float().numpy(), case["cache"], case["bt"], case["lens"], 2, D, pn["kc"],
                              pn["vc"], pn["R"], case["sm_scale"], "bfloat16")
    assert np.all(full[0] == 0)


def test_identical_keys_give_mean_of_values():
    case = identical_keys_case()
    pn = case["p"].np()
    got = O.decode_attention_rot(case["q"].float().numpy(), case["cache"], case["bt"], case["lens"], 2, D, pn["kc"],
                                 pn["vc"], pn["R"], case["sm_scale"], "bfloat16")[0]
    K, V = torch_dequant(case["cache"], case["bt"][0], 333, 2, pn["kc"], pn["vc"], cast=torch.bfloat16)
    assert torch.equal(K, K[0:1].expand_as(K))
    mean = V.mean(dim=0).numpy()  # (H, D)
    for h in range(8):
        assert rel_err(got[h], mean[h // 4]) < 1e-12


def test_roundings_match_torch_casts():
    """rotate_q == (q.float() @ R^T).to(bf16) and unrotate_out == (o.to(bf16).float() @ R).to(bf16),
    elementwise, on seeded data of the parity tests' scale."""
    for mode, iso_mode in (("iso", "fast"), ("iso", "full"), ("planar", "fast")):
        p = Params(mode, 3, 3, iso_mode=iso_mode)
        q = torch.randn(64, 32, D, generator=gen(46)).to(torch.bfloat16)
        got = O.rotate_q(q.float().numpy().reshape(-1, D), p.R.numpy(), "bfloat16")
        exp = (q.float().reshape(-1, D) @ p.R.T).to(torch.bfloat16).float().numpy()
        assert np.array_equal(got, exp), mode
        o = torch.randn(64 * 32, D, generator=gen(47), dtype=torch.float64) * 3
        got = O.unrotate_out(o.numpy(), p.R.numpy(), "bfloat16")
        exp = (o.to(torch.bfloat16).float() @ p.R).to(torch.bfloat16).float().numpy()
        assert np.array_equal(got, exp), mode


# ---------------------------------------------------------------------------
# Planted mistakes: each must fail at least one check above
# ---------------------------------------------------------------------------

def test_planted_gqa_map_is_caught(monkeypatch):
    monkeypatch.setattr(O, "_kv_head", lambda h, G, H: h % H)
    assert check_decode_vs_sdpa(_decode_case()) > 1e-3
    assert check_prefill_vs_sdpa(_prefill_case()) > 1e-3


@pytest.mark.parametrize("shift", [1, -1])
def test_planted_mask_offset_is_caught(monkeypatch, shift):
    orig = O._visible
    monkeypatch.setattr(O, "_visible", lambda pos, L: orig(np.asarray(pos) + shift, L))
    assert check_prefill_vs_sdpa(_prefill_case()) > 1e-3
    assert check_prefill_rows_are_prefix_decodes(_prefill_case()) > 1e-3


def test_planted_missing_scale_is_caught(monkeypatch):
    monkeypatch.setattr(O, "_scores", lambda qr, K, sm_scale: qr @ K.T)
    assert check_two_keys() > 1e-3
    assert check_decode_vs_sdpa(_decode_case()) > 1e-3


def test_planted_unrounded_kv_is_caught(monkeypatch):
    """K/V left as fp32 products (no cast to the q dtype) fail the decode and prefill checks."""
    monkeypatch.setattr(O, "decompress", lambda p, n, c, dt: O.decompress_f32(p, n, c))
    assert check_decode_vs_sdpa(_decode_case()) > 1e-4
    assert check_prefill_vs_sdpa(_prefill_case()) > 1e-4
    assert check_two_keys() > 1e-4


def test_fp32_kv_option_differs_from_the_default():
    """kv_dtype=None (no rounding) is an explicit option; the default rounds to the q dtype."""
    case = _decode_case()
    pn = case["p"].np()
    args = (case["q"].float().numpy(), case["cache"], case["bt"], case["lens"], case["H"], D, pn["kc"], pn["vc"],
            pn["R"], case["sm_scale"], "bfloat16")
    assert np.array_equal(O.decode_attention_rot(*args), O.decode_attention_rot(*args, kv_dtype="bfloat16"))
    assert not np.array_equal(O.decode_attention_rot(*args), O.decode_attention_rot(*args, kv_dtype=None))


# ---------------------------------------------------------------------------
# unfused_attention: the non-fused path (K/V decompressed to the q dtype)
# ---------------------------------------------------------------------------

def check_unfused_vs_sdpa(case, causal: bool) -> float:
    """unfused_attention_rot's math against float64 SDPA over K/V rounded by torch's
    own cast of the dequantized values (the pages flash attention reads)."""
    p = case["p"]
    pn = p.np()
    got = O.prefill_attention_rot(case["q"].float().numpy(), case["cu"], case["cache"], case["bt"], case["lens"],
                                  case["H"], D, pn["kc"], pn["vc"], pn["R"], case["sm_scale"], "bfloat16",
                                  causal=causal, kv_dtype="bfloat16")
    err = 0.0
    G = case["HQ"] // case["H"]
    for b in range(len(case["lens"])):
        s0, s1, L = int(case["cu"][b]), int(case["cu"][b + 1]), int(case["lens"][b])
        K, V = torch_dequant(case["cache"], case["bt"][b], L, case["H"], pn["kc"], pn["vc"])
        K, V = K.float().to(torch.bfloat16).double(), V.float().to(torch.bfloat16).double()
        qr = torch_q_rot(case["q"][s0:s1], p.R)
        T = s1 - s0
        pos = [L - T + i for i in range(T)] if causal else [L - 1] * T
        exp = sdpa_rot(qr, K, V, G, pos, case["sm_scale"]).numpy()
        err = max(err, rel_err(got[s0:s1], exp))
    return err


def check_unfused_noncausal_rows_are_decodes(case) -> float:
    """A non-causal row equals the decode oracle over the whole context (two code paths)."""
    p = case["p"]
    pn = p.np()
    args = (case["H"], D, pn["kc"], pn["vc"], pn["R"], case["sm_scale"], "bfloat16")
    full = O.prefill_attention_rot(case["q"].float().numpy(), case["cu"], case["cache"], case["bt"], case["lens"],
                                   *args, causal=False, kv_dtype="bfloat16")
    err = 0.0
    for b in range(len(case["lens"])):
        s0, s1, L = int(case["cu"][b]), int(case["cu"][b + 1]), int(case["lens"][b])
        for i in sorted({0, (s1 - s0) // 2, s1 - s0 - 1}):
            dec = O.decode_attention_rot(case["q"][s0 + i:s0 + i + 1].float().numpy(), case["cache"],
                                         case["bt"][b:b + 1], np.asarray([L]), *args, kv_dtype="bfloat16")
            err = max(err, rel_err(full[s0 + i], dec[0]))
    return err


def test_unfused_pages_equal_torch_cast():
    case = _prefill_case()
    pn = case["p"].np()
    L = int(case["lens"][0])
    K, V = O.gather_seq(case["cache"], case["bt"][0], L, case["H"], D, pn["kc"], pn["vc"], kv_dtype="bfloat16")
    Kt, Vt = torch_dequant(case["cache"], case["bt"][0], L, case["H"], pn["kc"], pn["vc"])
    assert np.array_equal(K, Kt.float().to(torch.bfloat16).double().numpy())
    assert np.array_equal(V, Vt.float().to(torch.bfloat16).double().numpy())


@pytest.mark.parametrize("causal", [True, False])
def test_unfused_matches_float64_sdpa(causal):
    assert check_unfused_vs_sdpa(_prefill_case(), causal) < 1e-10


def test_unfused_noncausal_rows_equal_decodes():
    assert check_unfused_noncausal_rows_are_decodes(_prefill_case()) < 1e-12


def test_unfused_entry_is_the_rounded_pages_path():
    """unfused_attention == prefill_attention with kv_dtype = the q dtype."""
    case = _prefill_case()
    pn = case["p"].np()
    args = (case["q"].float().numpy(), case["cu"], case["cache"], case["bt"], case["lens"], case["H"], D, pn["kc"],
            pn["vc"], pn["R"], case["sm_scale"], "bfloat16")
    assert np.array_equal(O.unfused_attention(*args, causal=False),
                          O.prefill_attention(*args, causal=False, kv_dtype="bfloat16"))


def test_planted_unrounded_pages_are_caught(monkeypatch):
    monkeypatch.setattr(O, "decompress", lambda p, n, c, dt: O.decompress_f32(p, n, c))
    assert check_unfused_vs_sdpa(_prefill_case(), True) > 1e-4


def test_planted_noncausal_truncation_is_caught(monkeypatch):
    """A non-causal mask that drops keys (here: the last 40) fails the SDPA check."""
    orig = O._visible
    monkeypatch.setattr(O, "_visible", lambda pos, L: orig(np.minimum(np.asarray(pos), L - 40), L))
    assert check_unfused_vs_sdpa(_prefill_case(), False) > 1e-3
