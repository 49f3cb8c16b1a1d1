"""RotorQuant KV-cache compression for vLLM on AMD Instinct MI355X (gfx950).

Drop-in for tpurtell/rotorquant-vllm's plugin surface (the CUSTOM attention
backend, RQ_* environment configuration and the packed uint8 cache layout),
with the hot path in hand-written HIP kernels behind a C ABI (librq_hip.so).

    # IsoQuant 3-bit (default)
    vllm serve <model> --attention-backend CUSTOM
    # PlanarQuant 4-bit / asymmetric K/V
    RQ_MODE=planar RQ_BITS=4 vllm serve <model> --attention-backend CUSTOM
    RQ_K_BITS=4 RQ_V_BITS=3 vllm serve <model> --attention-backend CUSTOM
"""
from rotorquant_vllm.quantization import IsoQuantMSE, LloydMaxCodebook, PlanarQuantMSE
from rotorquant_vllm.vllm import RQAttentionBackend, RQFullAttentionSpec, register_rq_backend

__all__ = [
    "IsoQuantMSE",
    "LloydMaxCodebook",
    "PlanarQuantMSE",
    "RQAttentionBackend",
    "RQFullAttentionSpec",
    "register_rq_backend",
]
