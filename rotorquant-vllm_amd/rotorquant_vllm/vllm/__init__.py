"""vLLM plugin surface: the CUSTOM attention backend and its KV spec.

Entry point (pyproject.toml): vllm.general_plugins -> rotorquant_vllm.vllm:register_rq_backend.
"""
from rotorquant_vllm.vllm.rq_backend import RQAttentionBackend, RQFullAttentionSpec, register_rq_backend

__all__ = ["RQAttentionBackend", "RQFullAttentionSpec", "register_rq_backend"]
