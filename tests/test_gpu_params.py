"""Rotation parameters built for a ROCm device, as vLLM builds them (device="cuda").

With RQ_PARAM_DEVICE unset (the default) the draws come from the CPU generator on
any target device, so q_L, q_R and rot2 on the GPU equal the golden fixture
(torch's CPU draws with the reference's seeds) bit for bit, and so does R.
With RQ_PARAM_DEVICE=device they come from the GPU's generator, as the reference
draws them on vLLM's device; this test prints whether those equal the CPU draws
(they need not: the result is the device RNG's) and checks only that they are
valid parameters.
"""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_cpu.npz"))


def test_default_draws_equal_cpu_fixture_on_gpu(monkeypatch):
    from rotorquant_vllm.quantization import IsoQuantMSE, PlanarQuantMSE
    from rotorquant_vllm.vllm.rq_backend import _build_rotation_matrix
    monkeypatch.delenv("RQ_PARAM_DEVICE", raising=False)
    iso = IsoQuantMSE(128, 3, seed=42, mode="full", device="cuda")
    pq = PlanarQuantMSE(128, 3, seed=42, device="cuda")
    assert iso.q_L.device.type == "cuda" and pq.rot2.device.type == "cuda"
    assert np.array_equal(iso.q_L.cpu().numpy().view(np.uint32), G["q_L"].view(np.uint32))
    assert np.array_equal(iso.q_R.cpu().numpy().view(np.uint32), G["q_R"].view(np.uint32))
    assert np.array_equal(pq.rot2.cpu().numpy().view(np.uint32), G["rot2"].view(np.uint32))
    R = _build_rotation_matrix(iso, 128, "cuda")
    assert np.array_equal(R.cpu().numpy().view(np.uint32), G["R_iso_full"].view(np.uint32))


def test_device_draws_are_valid_and_reported(monkeypatch):
    from rotorquant_vllm.quantization import IsoQuantMSE, PlanarQuantMSE
    monkeypatch.setenv("RQ_PARAM_DEVICE", "device")
    iso = IsoQuantMSE(128, 3, seed=42, mode="full", device="cuda")
    pq = PlanarQuantMSE(128, 3, seed=42, device="cuda")
    qL, rot2 = iso.q_L.cpu(), pq.rot2.cpu()
    assert torch.allclose(qL.norm(dim=-1), torch.ones(32), atol=1e-6)
    assert torch.allclose((rot2 ** 2).sum(-1), torch.ones(64), atol=1e-6)
    same_q = np.array_equal(qL.numpy().view(np.uint32), G["q_L"].view(np.uint32))
    same_r = np.array_equal(rot2.numpy().view(np.uint32), G["rot2"].view(np.uint32))
    print(f"RQ_PARAM_DEVICE=device on {torch.cuda.get_device_name()}: q_L equals the CPU draw: {same_q}; "
          f"rot2 equals the CPU draw: {same_r}", flush=True)
