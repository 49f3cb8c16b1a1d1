"""Import-path alias: the reference's op module name, backed by the HIP kernels.

Nothing in this package is Triton.  The reference's tests, benchmarks and users
import the op-level API from `rotorquant_vllm.triton`
(src/rotorquant_vllm/triton/__init__.py:1-15); this module keeps that path and
re-exports the same names from `rotorquant_vllm.kernels`, which calls the
gfx950 HIP library (librq_hip.so) through its C ABI.  The objects are the same
functions: `rotorquant_vllm.triton.fused_paged_rq_decode is
rotorquant_vllm.kernels.fused_paged_rq_decode`.
"""
from rotorquant_vllm.kernels import (
    fused_paged_rq_decode,
    fused_paged_rq_int8_prefill,
    iso_compress,
    iso_decompress,
    planar_compress,
    planar_decompress,
)

__all__ = [
    "iso_compress",
    "iso_decompress",
    "planar_compress",
    "planar_decompress",
    "fused_paged_rq_int8_prefill",
    "fused_paged_rq_decode",
]
