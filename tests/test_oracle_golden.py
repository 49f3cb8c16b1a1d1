"""Pin the CPU oracle and the init-time parameters (no GPU).

* rq_oracle.c vs the golden vectors of the reference's CPU path (bit-exact).
* rq_oracle.c vs the reference's torch op sequence at benchmark config-0 size.
* Lloyd-Max codebooks vs the scipy fixture, the closed form, and Max (1960).
* Rotation parameters / matrices vs the fixture and quaternion algebra.
"""
import math
import os

import numpy as np
import pytest
import torch

import oracle as O

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_cpu.npz"))
MODES = [("iso_fast", 4), ("iso_full", 4), ("planar", 2)]


def _rt(R):
    RT = R.T.copy()
    return np.ascontiguousarray(RT[:, 0::2]), np.ascontiguousarray(RT[:, 1::2])


@pytest.mark.parametrize("mode,blk", MODES)
@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("name,dt", [("f16", "float16"), ("bf16", "bfloat16")])
def test_oracle_matches_golden(mode, blk, bits, name, dt):
    re, ro = _rt(G[f"R_{mode}"])
    key = f"{mode}_b{bits}_{name}"
    p, n, _, n_ties = O.compress(G[f"x_{name}"], dt, re, ro, G[f"boundaries_b{bits}"], blk, want_ties=True)
    assert np.array_equal(p, G[f"packed_{key}"])
    assert np.array_equal(n.view(np.uint32), G[f"norms_{key}"].view(np.uint32))
    assert n_ties == int(G[f"ties_{key}"])
    dec = O.decompress(p, n, G[f"centroids_b{bits}"], dt)
    bits16 = (dec.view(np.uint32) >> 16).astype(np.uint16) if dt == "bfloat16" else dec.astype(np.float16).view(np.uint16)
    assert np.array_equal(bits16, G[f"dec_{key}"])


def test_planted_mistake_is_caught():
    """A plausible oracle slip (norm without the eps, or ties to the upper bucket) breaks the golden match."""
    re, ro = _rt(G["R_iso_fast"])
    x = G["x_f16"]
    b = G["boundaries_b4"]
    p_ok, _ = O.compress(x, "float16", re, ro, b, 4)
    # ties to the upper bucket (the Triton kernel's rule): move every boundary down one ulp
    p_up, _ = O.compress(x, "float16", re, ro, np.nextafter(b, -np.inf, dtype=np.float32), 4)
    assert np.array_equal(p_ok, G["packed_iso_fast_b4_f16"])
    assert not np.array_equal(p_up, G["packed_iso_fast_b4_f16"])
    # transposed rotation (R instead of R^T)
    re_t, ro_t = _rt(G["R_iso_fast"].T)
    p_t, _ = O.compress(x, "float16", re_t, ro_t, b, 4)
    assert not np.array_equal(p_t, G["packed_iso_fast_b4_f16"])


def test_oracle_matches_reference_ops_config0_full_size():
    """benchmark config 0: 2048 tokens x 8 heads x 128, K and V, iso fast 3-bit, vs the torch op sequence."""
    import make_golden as MG

    k, v = MG.config0_kv(2048, 0)
    R = torch.from_numpy(G["R_iso_fast"])
    RT = R.T.contiguous()
    rte, rto = RT[:, 0::2].contiguous(), RT[:, 1::2].contiguous()
    b = torch.from_numpy(G["boundaries_b3"])
    for x in (k, v):
        ref_p, ref_n, _, ties = MG.compress_cpu(x, rte, rto, b)
        p, n = O.compress(MG.bits16(x), "float16", rte.numpy(), rto.numpy(), b.numpy(), 4)
        assert np.array_equal(p, ref_p.numpy())
        assert np.array_equal(n.view(np.uint32), ref_n.numpy().view(np.uint32))


def test_codebooks_fixture_and_closed_form():
    from rotorquant_vllm.quantization import solve_lloyd_max
    from rotorquant_vllm.quantization.lloyd_max import lloyd_max_iterations

    for bits in (3, 4):
        c, b = solve_lloyd_max(128, bits)
        assert np.array_equal(c.numpy().view(np.uint32), G[f"centroids_b{bits}"].view(np.uint32))
        assert np.array_equal(b.numpy().view(np.uint32), G[f"boundaries_b{bits}"].view(np.uint32))
        cc, bc, it = O.lloyd_max_closed_form(128, bits)
        # every centroid agrees with the exact-integral iteration to the last fp32 bit
        assert np.array_equal(cc.astype(np.float32), c.numpy())
        mid = len(bc) // 2
        others = [i for i in range(len(bc)) if i != mid]
        assert np.array_equal(bc[others].astype(np.float32), b.numpy()[others])
        assert abs(float(b[mid])) < 1e-16 and abs(bc[mid]) < 1e-16
        assert it == lloyd_max_iterations(128, bits)
    # 3 bits converges (Max 1960 table, units of sigma); 4 bits stops at the 200-iteration cap
    assert lloyd_max_iterations(128, 3) == 138 and lloyd_max_iterations(128, 4) == 200
    c3, _ = solve_lloyd_max(128, 3)
    max1960 = np.array([0.2451, 0.7560, 1.3439, 2.1519])
    assert np.allclose(c3.numpy()[4:] * math.sqrt(128), max1960, atol=2e-4)
    assert np.array_equal(c3.numpy(), -c3.numpy()[::-1])


def test_middle_boundary_signs_decide_zero_vectors():
    """3-bit middle boundary is a tiny negative (zero lands in bucket 4); 4-bit is exactly 0 (tie -> bucket 7)."""
    assert G["boundaries_b3"][3] < 0 and G["boundaries_b3"][3] > -1e-16
    assert G["boundaries_b4"][7] == 0.0
    re, ro = _rt(G["R_iso_fast"])
    z = np.zeros((1, 1, 128), np.uint16)
    p3, _ = O.compress(z, "float16", re, ro, G["boundaries_b3"], 4)
    p4, _, _, t4 = O.compress(z, "float16", re, ro, G["boundaries_b4"], 4, want_ties=True)
    assert (p3 == 0x44).all() and (p4 == 0x77).all() and t4 == 128


def test_rotation_parameters():
    from rotorquant_vllm.quantization import IsoQuantMSE, PlanarQuantMSE
    from rotorquant_vllm.vllm.rq_backend import _build_iso_R, _build_planar_R

    iso = IsoQuantMSE(128, 3, seed=42, mode="full")
    assert np.array_equal(iso.q_L.numpy(), G["q_L"]) and np.array_equal(iso.q_R.numpy(), G["q_R"])
    assert np.allclose(np.linalg.norm(G["q_L"], axis=1), 1, atol=1e-6)
    pq = PlanarQuantMSE(128, 3, seed=42)
    assert np.array_equal(pq.rot2.numpy(), G["rot2"])
    assert np.allclose((G["rot2"] ** 2).sum(1), 1, atol=1e-6)
    for mode in ("fast", "full"):
        R = _build_iso_R(iso, 128, "cpu", mode).numpy()
        assert np.array_equal(R, G[f"R_iso_{mode}"])
    R = _build_planar_R(pq, 128, "cpu").numpy()
    assert np.array_equal(R, G["R_planar"])


def _quat_mul(a, b):
    aw, ax, ay, az = a
    bw, bx, by, bz = b
    return np.array([aw * bw - ax * bx - ay * by - az * bz, aw * bx + ax * bw + ay * bz - az * by,
                     aw * by - ax * bz + ay * bw + az * bx, aw * bz + ax * by - ay * bx + az * bw])


@pytest.mark.parametrize("mode", ["fast", "full"])
def test_iso_R_is_quaternion_sandwich(mode):
    """R block g maps v -> q_L v conj(q) with q = q_L (fast) or q_R (full), checked in float64."""
    qL, qR = G["q_L"].astype(np.float64), G["q_R"].astype(np.float64)
    R = G[f"R_iso_{mode}"].astype(np.float64)
    for g in range(32):
        q2 = qL[g] if mode == "fast" else qR[g]
        conj = q2 * np.array([1, -1, -1, -1])
        for e in range(4):
            v = np.eye(4)[e]
            img = _quat_mul(_quat_mul(qL[g], v), conj)
            assert np.allclose(R[4 * g:4 * g + 4, 4 * g + e], img, atol=2e-6)


@pytest.mark.parametrize("mode,blk", MODES)
def test_rotation_orthogonal_block_diagonal(mode, blk):
    """Reference test (tests/test_vllm_integration.py:94-105): max|R R^T - I| < 1e-5; off-block entries 0."""
    R = G[f"R_{mode}"].astype(np.float64)
    assert np.abs(R @ R.T - np.eye(128)).max() < 1e-5
    idx = np.arange(128)
    off = (idx[:, None] // blk) != (idx[None, :] // blk)
    assert (R[off] == 0).all()


def test_reference_cpu_ops_match_golden_and_c_oracle():
    """oracle.reference_cpu_compress / _decompress (the torch op sequence bench.py times
    as the compress CPU baseline) reproduce the golden vectors and the C restatement."""
    g = G
    for mode in ("iso_fast", "planar"):
        R = torch.from_numpy(g[f"R_{mode}"])
        RT = R.T.contiguous()
        rte, rto = RT[:, 0::2].contiguous(), RT[:, 1::2].contiguous()
        for bits in (3, 4):
            b = torch.from_numpy(g[f"boundaries_b{bits}"])
            c = torch.from_numpy(g[f"centroids_b{bits}"])
            x = torch.from_numpy(g["x_f16"].view(np.int16)).view(torch.float16)
            p_c, n_c = O.compress(g["x_f16"], "float16", rte.numpy(), rto.numpy(), b.numpy(), 4 if mode != "planar" else 2)
            packed, norms = O.reference_cpu_compress(x, rte, rto, b)
            key = f"{mode}_b{bits}_f16"
            assert np.array_equal(packed.numpy(), g[f"packed_{key}"]), key
            assert np.array_equal(packed.numpy(), p_c) and np.array_equal(norms.numpy(), n_c), key
            assert np.array_equal(norms.numpy().view(np.uint32), g[f"norms_{key}"].view(np.uint32)), key
            dec = O.reference_cpu_decompress(packed, norms, c, torch.float16)
            assert np.array_equal(dec.view(torch.int16).numpy().view(np.uint16), g[f"dec_{key}"]), key


def test_codebook_table_equals_the_solve():
    """The head_dim-128 codebooks returned from the fp32 table are bit-equal to the
    scipy solve on the reference's schedule and to the golden fixture."""
    from rotorquant_vllm.quantization import lloyd_max as LM
    for bits in (3, 4):
        c, b = LM.solve_lloyd_max(128, bits)
        cs, bs, _ = LM._solve(128, bits, False, 200, 1e-10)
        assert np.array_equal(c.numpy().view(np.uint32), np.asarray(cs, np.float32).view(np.uint32))
        assert np.array_equal(b.numpy().view(np.uint32), np.asarray(bs, np.float32).view(np.uint32))
        assert np.array_equal(c.numpy().view(np.uint32), G[f"centroids_b{bits}"].view(np.uint32))
        assert np.array_equal(b.numpy().view(np.uint32), G[f"boundaries_b{bits}"].view(np.uint32))


def test_param_device_env(monkeypatch):
    """RQ_PARAM_DEVICE: 'cpu' (default) draws on the CPU generator; bad values raise."""
    from rotorquant_vllm.quantization import IsoQuantMSE
    from rotorquant_vllm.quantization.lloyd_max import param_draw_device
    monkeypatch.delenv("RQ_PARAM_DEVICE", raising=False)
    assert param_draw_device("cuda").type == "cpu"
    monkeypatch.setenv("RQ_PARAM_DEVICE", "device")
    assert param_draw_device("cuda").type == "cuda"
    monkeypatch.setenv("RQ_PARAM_DEVICE", "gpu")
    with pytest.raises(ValueError, match="RQ_PARAM_DEVICE must be"):
        IsoQuantMSE(128, 3)


# ---------------------------------------------------------------------------
# Dense 3-bit index layout (opt-in; this build's own format)
# ---------------------------------------------------------------------------

def test_dense3_is_a_bit_permutation():
    """Each of the 96 input bits of a 32-index group (index i, bit b) lands on exactly
    one output bit, and no two on the same one: the layout loses nothing and
    needs exactly 3 bits per index."""
    seen = set()
    for i in range(32):
        for b in range(3):
            idx = np.zeros(32, np.uint8)
            idx[i] = 1 << b
            out = O.dense3_pack(O.indices_to_nibbles(idx))
            assert out.shape == (12,)
            bits = np.unpackbits(out, bitorder="little")
            assert bits.sum() == 1, (i, b)
            pos = int(np.flatnonzero(bits)[0])
            assert pos not in seen
            seen.add(pos)
    assert len(seen) == 96


def test_dense3_round_trip_every_value_at_every_position():
    rng = np.random.default_rng(5)
    idx = rng.integers(0, 8, (64, 8, 128), dtype=np.uint8)
    for v in range(8):  # every value at every position
        idx[v] = v
    nib = O.indices_to_nibbles(idx)
    dense = O.dense3_pack(nib)
    assert dense.shape == (64, 8, 48)
    assert np.array_equal(O.dense3_unpack(dense), nib)
    with pytest.raises(ValueError):
        O.dense3_pack(O.indices_to_nibbles(np.full(32, 8, np.uint8)))


def test_dense3_slot_layout_and_cache_round_trip():
    lay = O.slot_layout(8, 128, dense3=True)
    assert (lay["index_bytes"], lay["k_idx_end"], lay["k_norm_end"], lay["v_idx_end"], lay["v_norm_end"],
            lay["total_bytes"]) == (48, 384, 416, 800, 832, 1024)
    from rotorquant_vllm.vllm.rq_backend import _rq_total_bytes
    assert _rq_total_bytes(128, 8, dense3=True) == 1024 and _rq_total_bytes(128, 8) == 2048
    rng = np.random.default_rng(6)
    N, H = 40, 4
    kp = O.indices_to_nibbles(rng.integers(0, 8, (N, H, 128), dtype=np.uint8))
    vp = O.indices_to_nibbles(rng.integers(0, 8, (N, H, 128), dtype=np.uint8))
    kn = rng.standard_normal((N, H, 1)).astype(np.float32)
    vn = rng.standard_normal((N, H, 1)).astype(np.float32)
    cache = np.zeros((4, 16, O.slot_layout(H, 128, True)["total_bytes"]), np.uint8)
    slots = rng.permutation(64)[:N]
    O.compress_store(cache, slots, kp, kn, vp, vn, dense3=True)
    rkp, rkn, rvp, rvn = O.read_slots(cache, H, 128, dense3=True)
    assert np.array_equal(rkp[slots], kp) and np.array_equal(rvp[slots], vp)
    assert np.array_equal(rkn[slots], kn) and np.array_equal(rvn[slots], vn)
    nib = O.dense3_cache_to_nibbles(cache, H, 128)
    ref = np.zeros((4, 16, O.slot_layout(H, 128)["total_bytes"]), np.uint8)
    O.compress_store(ref, np.arange(64), rkp, rkn, rvp, rvn)
    assert np.array_equal(nib, ref)
