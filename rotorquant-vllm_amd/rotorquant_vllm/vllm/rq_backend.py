"""RotorQuant compressed-KV attention backend for vLLM, on gfx950 HIP kernels.

Drop-in for the reference plugin (src/rotorquant_vllm/vllm/rq_backend.py): same
registration (`register_rq_backend`, the CUSTOM backend), the same RQ_* env
configuration, the same packed uint8 (num_blocks, block_size, total_bytes)
cache with per-token slots

    [K idx (H x D/2) | K norms (H x fp32) | V idx | V norms | zero pad to H * next_pow2(D + 8)]

and the same class / attribute names, so the reference's fake-based dispatch
tests run unchanged against it.  The hot path underneath is the C ABI of
librq_hip.so (include/rq_abi.h):

    compress + store  -> rq_compress_store   (one fused K+V launch, writes slots)
    decode            -> rq_fused_decode     (Q and output rotation inside)
    prefill           -> rq_int8_prefill     (int8 MFMA, multi-sequence)
    non-fused path    -> rq_paged_attention  (K/V dequantized to the q dtype in
                         LDS, 16-bit MFMA; head_size 128; decodes), and for
                         longer queries rq_paged_prefill (the same arithmetic,
                         each tile decoded once); other head sizes
                         rq_paged_decompress + device attention in fp32

vLLM itself is imported lazily: without vLLM the module still imports (the
classes then derive from small local stand-ins), which is how the tests run.
"""
from __future__ import annotations

import enum
import functools
import inspect
import logging
import os
from dataclasses import dataclass
from dataclasses import fields as dc_fields
from fractions import Fraction

import numpy as np
import torch

from rotorquant_vllm.quantization.isoquant import IsoQuantMSE
from rotorquant_vllm.quantization.planarquant import PlanarQuantMSE

logger = logging.getLogger(__name__)

# ---------------------------------------------------------------------------
# Constants (reference: rq_backend.py:51-54)
# ---------------------------------------------------------------------------

RQ_DEFAULT_BITS = 3
RQ_DEFAULT_MODE = "iso"
RQ_SEED = 42
RQ_NORM_BYTES = 4

# ---------------------------------------------------------------------------
# Env parsing (reference: rq_backend.py:62-109, :140-148); same messages
# ---------------------------------------------------------------------------


def _parse_rq_mode() -> str:
    mode = os.environ.get("RQ_MODE", RQ_DEFAULT_MODE).lower()
    if mode not in ("iso", "planar"):
        raise ValueError(f"RQ_MODE must be 'iso' or 'planar', got '{mode}'")
    return mode


def _parse_rq_bits() -> int:
    bits = int(os.environ.get("RQ_BITS", str(RQ_DEFAULT_BITS)))
    if bits not in (3, 4):
        raise ValueError(f"RQ_BITS must be 3 or 4, got '{bits}'")
    return bits


def _parse_kv_bits() -> tuple[int, int]:
    default = _parse_rq_bits()
    k_raw, v_raw = os.environ.get("RQ_K_BITS"), os.environ.get("RQ_V_BITS")
    k_bits = int(k_raw) if k_raw else default
    v_bits = int(v_raw) if v_raw else default
    if k_bits not in (3, 4):
        raise ValueError(f"RQ_K_BITS must be 3 or 4, got '{k_bits}'")
    if v_bits not in (3, 4):
        raise ValueError(f"RQ_V_BITS must be 3 or 4, got '{v_bits}'")
    return k_bits, v_bits


def _parse_dense3() -> bool:
    """RQ_DENSE_3BIT=1 (opt-in, no counterpart in the reference): the dense 3-bit index
    layout, 3 D / 8 index bytes per head instead of D / 2 (RQ_INDEX_DENSE3 in
    include/rq_abi.h).  It holds 3-bit indices only."""
    on = os.environ.get("RQ_DENSE_3BIT", "").lower() in ("1", "true", "yes")
    if on and _parse_kv_bits() != (3, 3):
        raise ValueError("RQ_DENSE_3BIT needs 3-bit K and V (RQ_BITS=3, RQ_K_BITS / RQ_V_BITS unset or 3)")
    return on


def _parse_iso_mode() -> str:
    mode = os.environ.get("RQ_ISO_MODE", "fast").lower()
    if mode not in ("fast", "full"):
        raise ValueError(f"RQ_ISO_MODE must be 'fast' or 'full', got '{mode}'")
    return mode


def _parse_rq_fused_paged_env() -> bool:
    return os.environ.get("RQ_USE_FUSED_PAGED", "").lower() in ("1", "true", "yes")


# ---------------------------------------------------------------------------
# Kernel feature gates (reference: rq_backend.py:118-138): on if librq_hip.so loads
# ---------------------------------------------------------------------------

_fused_paged_kernel_available = False
_fused_prefill_kernel_available = False
_fused_paged_rq_decode_fn = None
_fused_paged_rq_int8_prefill_fn = None
_compress_store_fn = None
_paged_decompress_fn = None
_paged_attention_fn = None
_paged_prefill_fn = None
_unfused_decode_fn = None
_shared_workspace = None
try:
    from rotorquant_vllm import _lib as _rq_lib
    from rotorquant_vllm.kernels import compress_store as _compress_store_fn
    from rotorquant_vllm.kernels import fused_paged_rq_decode as _fused_paged_rq_decode_fn
    from rotorquant_vllm.kernels import fused_paged_rq_int8_prefill as _fused_paged_rq_int8_prefill_fn
    from rotorquant_vllm.kernels import paged_attention as _paged_attention_fn
    from rotorquant_vllm.kernels import paged_prefill as _paged_prefill_fn
    # The non-fused path's single-token decodes (a separate hook from the fused path's)
    from rotorquant_vllm.kernels import fused_paged_rq_decode as _unfused_decode_fn
    from rotorquant_vllm.kernels import paged_decompress as _paged_decompress_fn
    from rotorquant_vllm.kernels import shared_workspace as _shared_workspace

    _rq_lib.load()
    _fused_paged_kernel_available = True
    _fused_prefill_kernel_available = True
except (ImportError, OSError, RuntimeError) as exc:
    logger.info("RotorQuant HIP kernels unavailable: %s", exc)

# Queries of at most this many tokens take the non-fused path's one-launch kernel
# (rq_paged_attention: one query block per (sequence, kv head), each tile decoded
# once anyway); longer ones take rq_paged_prefill, which decodes each tile once
# for all query blocks instead of once per block.
RQ_UNFUSED_SHORT_Q = 16

# Shapes the fused kernels take (checked again by the C ABI): head_dim 128, a
# GQA group of at most 16 query heads, at most 64 kv heads.
RQ_FUSED_HEAD_DIM = 128
RQ_FUSED_MAX_GQA = 16
RQ_FUSED_MAX_KV_HEADS = 64


def _fused_shape_ok(num_heads: int, num_kv_heads: int, head_size: int) -> str | None:
    """None if the fused kernels take this attention shape, else the reason they do not."""
    if head_size != RQ_FUSED_HEAD_DIM:
        return f"head_size {head_size} (the fused kernels take {RQ_FUSED_HEAD_DIM})"
    if num_kv_heads < 1 or num_kv_heads > RQ_FUSED_MAX_KV_HEADS:
        return f"{num_kv_heads} kv heads (at most {RQ_FUSED_MAX_KV_HEADS})"
    if num_heads % num_kv_heads or num_heads // num_kv_heads > RQ_FUSED_MAX_GQA:
        return f"{num_heads} query heads over {num_kv_heads} kv heads (GQA group must be an integer <= 16)"
    return None


@functools.lru_cache(maxsize=64)
def _accepted_keywords(fn) -> frozenset | None:
    """Keyword names fn accepts (None: any).  The module-level kernel hooks below are
    monkey-patchable, and a replacement may have the reference's narrower signature
    (fused_paged_rq_decode.py:214-227, fused_paged_rq_int8_prefill.py:247-260)."""
    try:
        params = inspect.signature(fn).parameters
    except (TypeError, ValueError):
        return frozenset()
    if any(p.kind is inspect.Parameter.VAR_KEYWORD for p in params.values()):
        return None
    return frozenset(params)


def _call_hook(fn, *args, **kwargs):
    """fn(*args, **kwargs) with the keyword arguments fn does not accept left out; only
    the optional extras of this build (workspace, max_seq_len, cu_seqlens_q, max_q_len)
    are ever dropped: the reference's own keywords are accepted by every hook.  A hook
    that cannot read the dense 3-bit layout is refused when the cache holds it."""
    names = _accepted_keywords(fn)
    if names is not None:
        if kwargs.get("dense3") and "dense3" not in names:
            raise RuntimeError(f"{getattr(fn, '__name__', fn)} does not take the dense 3-bit cache (RQ_DENSE_3BIT)")
        kwargs = {k: v for k, v in kwargs.items() if k in names}
    return fn(*args, **kwargs)


# ---------------------------------------------------------------------------
# Cache size helpers (reference: rq_backend.py:155-188)
# ---------------------------------------------------------------------------


def _next_power_of_2(n: int) -> int:
    return 1 << (n - 1).bit_length() if n > 0 else 1


def _rq_index_bytes(head_dim: int, dense3: bool = False) -> int:
    """Index bytes per head: nibbles (head_dim / 2), or the dense 3-bit layout (3 head_dim / 8)."""
    return 3 * head_dim // 8 if dense3 else head_dim // 2


def _rq_bytes_per_component(head_dim: int, num_kv_heads: int, dense3: bool = False) -> int:
    """Packed indices plus one fp32 norm, per head."""
    return num_kv_heads * _rq_index_bytes(head_dim, dense3) + num_kv_heads * RQ_NORM_BYTES


def _rq_bytes_per_token_kv(head_dim: int, num_kv_heads: int, dense3: bool = False) -> int:
    """K + V payload per token (1088 B for 8 heads of 128; 832 B in the dense 3-bit layout)."""
    return 2 * _rq_bytes_per_component(head_dim, num_kv_heads, dense3)


def _rq_padded_slot_bytes(head_dim: int, dense3: bool = False) -> int:
    """Per-head slot share, padded to a power of two (256 B for head_dim 128; dense 3-bit: 128 B)."""
    return _next_power_of_2(_rq_bytes_per_token_kv(head_dim, 1, dense3))


def _rq_total_bytes(head_dim: int, num_kv_heads: int, dense3: bool = False) -> int:
    return num_kv_heads * _rq_padded_slot_bytes(head_dim, dense3)


# ---------------------------------------------------------------------------
# Rotation matrices (reference: rq_backend.py:194-264)
# ---------------------------------------------------------------------------


def _quat_left(w, x, y, z) -> torch.Tensor:
    """Matrix of v -> q v (Hamilton product, [w, x, y, z] order)."""
    return torch.tensor([[w, -x, -y, -z],
                         [x, w, -z, y],
                         [y, z, w, -x],
                         [z, -y, x, w]], dtype=torch.float32)


def _quat_right_conj(w, x, y, z) -> torch.Tensor:
    """Matrix of v -> v conj(q)."""
    return torch.tensor([[w, x, y, z],
                         [-x, w, -z, y],
                         [-y, z, w, -x],
                         [-z, -y, x, w]], dtype=torch.float32)


def _round_f32(x: Fraction) -> float:
    """x rounded to the nearest fp32 value (ties to even), from its exact value."""
    c = np.float32(float(x))  # within one fp32 ulp of the answer
    best = None
    for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        key = (abs(Fraction(float(cand)) - x), int(np.asarray(cand, np.float32).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, float(cand))
    return best[1]


def _block_product_f32(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """A @ B for small fp32 blocks in one fixed order: entry (i, j) is the fma chain
    over k = 1, 2, ... starting from the rounded product A[i,0] * B[0,j], each step
    computed exactly and rounded once.  That is the order of the fp32 sgemm that
    produced the reference-side fixture (MKL on AVX-512); evaluated this way the
    result is the same on every host and device, where torch's own matmul differs
    by BLAS path."""
    a = [[Fraction(float(v)) for v in row] for row in A.tolist()]
    b = [[Fraction(float(v)) for v in row] for row in B.tolist()]
    n, m, kk = len(a), len(b[0]), len(b)
    out = torch.empty(n, m, dtype=torch.float32)
    for i in range(n):
        for j in range(m):
            acc = _round_f32(a[i][0] * b[0][j])
            for k in range(1, kk):
                acc = _round_f32(a[i][k] * b[k][j] + Fraction(acc))
            out[i, j] = acc
    return out


_iso_R_cache: dict = {}


def _build_iso_R(quantizer, d: int, device, mode: str = "fast") -> torch.Tensor:
    """Block-diagonal R with 4x4 blocks: 'fast' v -> q_L v conj(q_L), 'full' v -> q_L v conj(q_R).

    The fp32 4x4 block products (init-time, 32 blocks) are formed in a fixed
    order on the host (_block_product_f32) and R is then moved to `device`, so R
    and every cache byte written with it are the same on any machine.
    """
    qL = quantizer.q_L.detach().float().cpu()
    qR = quantizer.q_R.detach().float().cpu() if mode == "full" else qL
    D_pad = quantizer.d_padded
    key = (d, D_pad, qL.numpy().tobytes(), qR.numpy().tobytes())
    R = _iso_R_cache.get(key)  # every layer draws the same seeded parameters
    if R is None:
        R = torch.eye(D_pad, dtype=torch.float32)
        for g in range(quantizer.n_groups):
            lw, lx, ly, lz = (float(v) for v in qL[g])
            rw, rx, ry, rz = (float(v) for v in qR[g])
            R[4 * g:4 * g + 4, 4 * g:4 * g + 4] = _block_product_f32(_quat_left(lw, lx, ly, lz),
                                                                     _quat_right_conj(rw, rx, ry, rz))
        R = R[:d, :d].contiguous()
        _iso_R_cache[key] = R
    return R.clone().to(device)


def _build_planar_R(quantizer, d: int, device) -> torch.Tensor:
    """Block-diagonal R with 2x2 Givens blocks [[c, -s], [s, c]]."""
    cs = quantizer.rot2.detach().float().cpu()
    R = torch.eye(quantizer.d_padded, dtype=torch.float32)
    for g in range(quantizer.n_groups):
        c, s = float(cs[g, 0]), float(cs[g, 1])
        R[2 * g:2 * g + 2, 2 * g:2 * g + 2] = torch.tensor([[c, -s], [s, c]], dtype=torch.float32)
    return R[:d, :d].contiguous().to(device)


def _build_rotation_matrix(quantizer, d: int, device) -> torch.Tensor:
    if hasattr(quantizer, "q_L"):
        return _build_iso_R(quantizer, d, device, getattr(quantizer, "mode", "fast"))
    return _build_planar_R(quantizer, d, device)


# ---------------------------------------------------------------------------
# vLLM base classes (lazy; local stand-ins when vLLM is absent)
# ---------------------------------------------------------------------------


class _AttentionTypeStandIn(str, enum.Enum):
    DECODER = "decoder"
    ENCODER = "encoder"
    ENCODER_ONLY = "encoder_only"
    ENCODER_DECODER = "encoder_decoder"


class _CGSupportStandIn(enum.Enum):
    NEVER = 0
    UNIFORM_SINGLE_TOKEN_DECODE = 1
    UNIFORM_BATCH = 2
    ALWAYS = 3


class _BackendStandIn:
    pass


class _ImplStandIn:
    def __init__(self, num_heads, head_size, scale, num_kv_heads=None, alibi_slopes=None, sliding_window=None,
                 kv_cache_dtype="auto", logits_soft_cap=None, attn_type=_AttentionTypeStandIn.DECODER,
                 *args, **kwargs):
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.num_kv_heads = num_kv_heads if num_kv_heads is not None else num_heads
        self.alibi_slopes = alibi_slopes
        self.sliding_window = sliding_window
        self.kv_cache_dtype = kv_cache_dtype
        self.logits_soft_cap = logits_soft_cap
        self.attn_type = attn_type


class _BuilderStandIn:
    pass


@dataclass(frozen=True, kw_only=True)
class _FullAttentionSpecStandIn:
    block_size: int
    num_kv_heads: int
    head_size: int
    dtype: torch.dtype


def _import_vllm_bases():
    """Best available vLLM base classes: FlashAttention* (as the reference), ROCm's, or stand-ins."""
    try:
        from vllm.v1.attention.backend import AttentionCGSupport, AttentionType
    except Exception:  # noqa: BLE001  (vLLM absent or incompatible)
        return (_BackendStandIn, _ImplStandIn, _BuilderStandIn, _FullAttentionSpecStandIn,
                _CGSupportStandIn, _AttentionTypeStandIn, False)
    try:
        from vllm.v1.kv_cache_interface import FullAttentionSpec
    except Exception:  # noqa: BLE001
        FullAttentionSpec = _FullAttentionSpecStandIn
    for mod, names in (("vllm.v1.attention.backends.flash_attn",
                        ("FlashAttentionBackend", "FlashAttentionImpl", "FlashAttentionMetadataBuilder")),
                       ("vllm.v1.attention.backends.rocm_attn",
                        ("RocmAttentionBackend", "RocmAttentionImpl", "RocmAttentionMetadataBuilder")),
                       ("vllm.v1.attention.backends.triton_attn",
                        ("TritonAttentionBackend", "TritonAttentionImpl", "TritonAttentionMetadataBuilder"))):
        try:
            m = __import__(mod, fromlist=list(names))
            return (getattr(m, names[0]), getattr(m, names[1]), getattr(m, names[2]), FullAttentionSpec,
                    AttentionCGSupport, AttentionType, True)
        except Exception:  # noqa: BLE001
            continue
    return (_BackendStandIn, _ImplStandIn, _BuilderStandIn, FullAttentionSpec, AttentionCGSupport, AttentionType,
            True)


(_BackendBase, _ImplBase, _BuilderBase, FullAttentionSpec, AttentionCGSupport, AttentionType,
 _HAVE_VLLM) = _import_vllm_bases()

# ---------------------------------------------------------------------------
# KV cache spec (reference: rq_backend.py:272-283)
# ---------------------------------------------------------------------------


@dataclass(frozen=True, kw_only=True)
class RQFullAttentionSpec(FullAttentionSpec):
    """Full-attention KV spec whose pages hold the packed RotorQuant slots (uint8)."""

    @property
    def real_page_size_bytes(self) -> int:  # noqa: D102
        return self.block_size * _rq_total_bytes(self.head_size, self.num_kv_heads, _parse_dense3())


# ---------------------------------------------------------------------------
# Metadata builder (reference: rq_backend.py:291-313)
# ---------------------------------------------------------------------------


class RQMetadataBuilder(_BuilderBase):
    """Builder of the parent backend; HIP-graph capture of uniform single-token decode
    batches whenever the kernels take the shape (the fused decode and the non-fused
    rq_paged_attention both launch with sizes independent of the context lengths).

    Two additions to the parent's metadata, both for mixed batches:
    * reorder_batch_threshold = 1 asks vLLM's model runner to put single-token
      (decode) requests first, so a mixed batch is [decodes | prefill chunks]
      and each part is a contiguous range of sequences;
    * the host copies of query_start_loc and seq_lens that vLLM already holds
      (CommonAttentionMetadata.query_start_loc_cpu / seq_lens_cpu) are attached
      as rq_query_start_loc_cpu / rq_seq_lens_cpu, so forward() splits and
      groups a mixed batch without reading device memory.
    """

    reorder_batch_threshold = 1

    @classmethod
    def get_cudagraph_support(cls, vllm_config: object, kv_cache_spec: object):
        """UNIFORM_SINGLE_TOKEN_DECODE when the layer's decodes run a HIP kernel whose
        launch does not depend on host data (the fused decode, or rq_paged_attention):
        the library loads, head_size 128, a GQA group the kernels take and an f16 /
        bf16 model.  Otherwise NEVER: such decodes run the torch fallback, whose loop
        over host lengths cannot be captured."""
        if not _fused_paged_kernel_available:
            return AttentionCGSupport.NEVER
        head_size = getattr(kv_cache_spec, "head_size", RQ_FUSED_HEAD_DIM)
        if head_size != RQ_FUSED_HEAD_DIM:
            return AttentionCGSupport.NEVER
        model_config = getattr(vllm_config, "model_config", None)
        dtype = getattr(model_config, "dtype", None)
        if isinstance(dtype, torch.dtype) and dtype not in (torch.float16, torch.bfloat16):
            return AttentionCGSupport.NEVER
        num_kv = getattr(kv_cache_spec, "num_kv_heads", None)
        num_heads = None
        try:
            num_heads = model_config.get_num_attention_heads(vllm_config.parallel_config)
        except Exception:  # no model config (tests) or an older vLLM: decided by head_size alone
            pass
        if num_kv and num_heads and _fused_shape_ok(num_heads, num_kv, head_size) is not None:
            return AttentionCGSupport.NEVER
        return AttentionCGSupport.UNIFORM_SINGLE_TOKEN_DECODE

    def build(self, *args, **kwargs):  # noqa: D102
        md = super().build(*args, **kwargs)
        common = kwargs.get("common_attn_metadata", args[1] if len(args) > 1 else None)
        for name in ("query_start_loc_cpu", "seq_lens_cpu"):
            val = getattr(common, name, None)
            if val is not None:
                try:
                    setattr(md, "rq_" + name, val)
                except (AttributeError, TypeError):  # frozen / slotted metadata: forward reads device copies
                    pass
        return md


# ---------------------------------------------------------------------------
# Backend (reference: rq_backend.py:322-371)
# ---------------------------------------------------------------------------


class RQAttentionBackend(_BackendBase):
    """RotorQuant compressed-KV attention backend, registered as CUSTOM."""

    forward_includes_kv_cache_update = True

    @classmethod
    def supports_mm_prefix(cls) -> bool:
        return True

    @staticmethod
    def get_name() -> str:
        return "CUSTOM"

    @staticmethod
    def get_impl_cls():
        return RQAttentionImpl

    @staticmethod
    def get_builder_cls():
        return RQMetadataBuilder

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int,
                           cache_dtype_str: str = "auto") -> tuple[int, ...]:
        """(num_blocks, block_size, total_bytes) uint8."""
        return (num_blocks, block_size, _rq_total_bytes(head_size, num_kv_heads, _parse_dense3()))

    @staticmethod
    def get_kv_cache_stride_order(include_num_layers_dimension: bool = False) -> tuple[int, ...]:
        """Raises so vLLM falls back to the identity layout."""
        raise NotImplementedError


# ---------------------------------------------------------------------------
# Attention implementation (reference: rq_backend.py:379-1036)
# ---------------------------------------------------------------------------


class RQAttentionImpl(_ImplBase):
    """compress -> store -> fused decode / int8 prefill (or paged decompress + attention)."""

    def __init__(self, *args, **kwargs) -> None:
        super().__init__(*args, **kwargs)
        head_size = self.head_size
        num_kv_heads = self.num_kv_heads
        rq_mode = _parse_rq_mode()
        iso_mode = _parse_iso_mode()
        k_bits, v_bits = _parse_kv_bits()
        self._k_bits, self._v_bits, self._rq_mode = k_bits, v_bits, rq_mode

        vllm_config = None
        if _HAVE_VLLM:
            try:
                from vllm.config import get_current_vllm_config_or_none
                vllm_config = get_current_vllm_config_or_none()
            except Exception:  # noqa: BLE001
                vllm_config = None
        device = vllm_config.device_config.device if vllm_config is not None else torch.device("cpu")

        if rq_mode == "iso":
            kq = IsoQuantMSE(head_size, k_bits, seed=RQ_SEED, mode=iso_mode, device=device)
            vq = kq if v_bits == k_bits else IsoQuantMSE(head_size, v_bits, seed=RQ_SEED, mode=iso_mode,
                                                         device=device)
        else:
            kq = PlanarQuantMSE(head_size, k_bits, seed=RQ_SEED, device=device)
            vq = kq if v_bits == k_bits else PlanarQuantMSE(head_size, v_bits, seed=RQ_SEED, device=device)
        self._k_quantizer, self._v_quantizer = kq, vq

        # One R (from the K quantizer) serves K and V (reference :472-480).
        R = _build_rotation_matrix(kq, head_size, device)
        self._rq_rot = R
        self._rq_rot_T = R.T.contiguous()
        self._rq_rot_T_even = self._rq_rot_T[:, 0::2].contiguous()
        self._rq_rot_T_odd = self._rq_rot_T[:, 1::2].contiguous()
        self._rq_rot_block = 4 if rq_mode == "iso" else 2
        self._half_d = head_size // 2
        self._dense3 = _parse_dense3()
        if self._dense3 and head_size % 32:
            raise ValueError(f"RQ_DENSE_3BIT needs head_size % 32 == 0 (got {head_size})")
        ib = _rq_index_bytes(head_size, self._dense3)

        self._k_idx_end = num_kv_heads * ib
        self._k_norm_end = self._k_idx_end + num_kv_heads * RQ_NORM_BYTES
        self._v_idx_end = self._k_norm_end + num_kv_heads * ib
        self._v_norm_end = self._v_idx_end + num_kv_heads * RQ_NORM_BYTES
        self._total_bytes = _rq_total_bytes(head_size, num_kv_heads, self._dense3)

        self._cg_buffers_ready = False
        self._max_model_len = vllm_config.model_config.max_model_len if vllm_config is not None else 8192
        self._max_prefill_len = (vllm_config.scheduler_config.max_num_batched_tokens
                                 if vllm_config is not None else 2048)
        self._max_num_seqs = (getattr(vllm_config.scheduler_config, "max_num_seqs", 256)
                              if vllm_config is not None else 256)
        env_on = _parse_rq_fused_paged_env()
        why_not = _fused_shape_ok(self.num_heads, num_kv_heads, head_size)
        if env_on and why_not is not None:
            logger.info("RotorQuant fused kernels off for this layer: %s", why_not)
        self._fused_paged_available = env_on and _fused_paged_kernel_available and why_not is None
        self._fused_prefill_available = env_on and _fused_prefill_kernel_available and why_not is None

        fp16_total = 2 * num_kv_heads * head_size * 2
        logger.info("RQAttentionImpl: %s mode, %d KV heads, head_size=%d, k_bits=%d, v_bits=%d, "
                    "%d bytes/token (%.2fx compression vs FP16)", rq_mode, num_kv_heads, head_size, k_bits,
                    v_bits, self._total_bytes, fp16_total / self._total_bytes)
        logger.info("Fused paged RQ decode: %s; fused paged RQ int8 prefill: %s",
                    "enabled" if self._fused_paged_available else "disabled",
                    "enabled" if self._fused_prefill_available else "disabled")

    # -- scratch -----------------------------------------------------------

    def _init_cg_buffers(self, kv_cache, compute_dtype):
        """Device tensors every launch reads (codebooks, R and its R^T splits), and the
        shared workspaces sized for the largest call this configuration allows
        (max_num_seqs sequences of max_model_len for decode, one max_model_len
        sequence of tile images for prefill).  This runs at the first forward --
        vLLM's profiling run -- so later calls find their scratch allocated; the
        workspaces are shared by all layers of the process on this device and are
        never freed (rotorquant_vllm.kernels.shared_workspace)."""
        dev = kv_cache.device
        self._dev_kc = self._k_quantizer.centroids.to(dev, torch.float32).contiguous()
        self._dev_vc = self._v_quantizer.centroids.to(dev, torch.float32).contiguous()
        self._dev_kb = self._k_quantizer.boundaries.to(dev, torch.float32).contiguous()
        self._dev_vb = self._v_quantizer.boundaries.to(dev, torch.float32).contiguous()
        self._dev_R = self._rq_rot.to(dev, torch.float32).contiguous()
        self._dev_rte = self._rq_rot_T_even.to(dev, torch.float32).contiguous()
        self._dev_rto = self._rq_rot_T_odd.to(dev, torch.float32).contiguous()
        if dev.type == "cuda" and _shared_workspace is not None:
            lib = _rq_lib.load()
            cap = -(-self._max_model_len // kv_cache.shape[1]) * kv_cache.shape[1]
            unfused_decode = _unfused_decode_fn is not None and self._unfused_kernel_ok(compute_dtype, self.num_heads)
            if self._fused_paged_available or unfused_decode:
                _shared_workspace(dev, "decode", lib.rq_fused_decode_workspace_bytes(
                    self._max_num_seqs, self.num_heads, self.head_size, cap))
            if self._fused_prefill_available or self._unfused_kernel_ok(compute_dtype, self.num_heads):
                _shared_workspace(dev, "prefill", lib.rq_int8_prefill_workspace_bytes(1, self.num_kv_heads, cap))
        self._cg_buffers_ready = True

    def _layout_kw(self) -> dict:
        """{"dense3": True} when the cache holds the dense 3-bit layout; else nothing, so
        the kernel hooks are called exactly as the reference calls them."""
        return {"dense3": True} if getattr(self, "_dense3", False) else {}

    def _launch_operands(self):
        """(K centroids, V centroids, R) for the kernel hooks: the device copies once
        _init_cg_buffers ran, else the quantizers' own tensors."""
        if hasattr(self, "_dev_kc"):
            return self._dev_kc, self._dev_vc, self._dev_R
        return self._k_quantizer.centroids, self._v_quantizer.centroids, self._rq_rot

    # -- compress + store ----------------------------------------------------

    def _compress_and_store(self, key, value, kv_cache, slot_mapping, compress_out=None, row_out=None) -> None:
        """Fused K+V compress written straight into the slots (rq_backend.py:585-657)."""
        if _compress_store_fn is None:
            raise RuntimeError("RotorQuant HIP kernels are not available")
        n = slot_mapping.shape[0]
        _compress_store_fn(key[:n], value[:n], kv_cache, slot_mapping, self._dev_rte, self._dev_rto,
                           self._dev_kb, self._dev_vb, rot_block=self._rq_rot_block, **self._layout_kw())

    # -- fused paths -----------------------------------------------------------

    def _fused_decode(self, query, kv_cache, block_table, seq_lens, output, n, fn=None):
        """Fused decode of sequences [0, n) (one query token each) into output[:n], through
        fn (default: the fused path's hook _fused_paged_rq_decode_fn).

        max_seq_len is the block table's capacity, not the batch's longest
        sequence: a captured HIP graph replays with longer sequences than it was
        captured with, so the launch must not depend on the lengths."""
        fn = _fused_paged_rq_decode_fn if fn is None else fn
        kc, vc, R = self._launch_operands()
        BS = kv_cache.shape[1]
        cap = block_table.shape[1] * BS
        ws = None
        if _shared_workspace is not None and query.device.type == "cuda":
            ws = _shared_workspace(query.device, "decode", _rq_lib.load().rq_fused_decode_workspace_bytes(
                n, query.shape[1], self.head_size, cap))
        _call_hook(fn, query[:n], kv_cache, block_table, seq_lens, kc, vc, R,
                   self.num_kv_heads, self.head_size, BS, sm_scale=self.scale, out=output[:n], max_seq_len=cap,
                   workspace=ws, **self._layout_kw())

    def _prefill_groups(self, lens: list, q_lens: list, b0: int, BS: int, max_blocks: int, device):
        """Split sequences [b0, B) into contiguous groups whose tile images fit the
        prefill workspace (sized at init for one max_model_len sequence):
        [(b_start, b_end, max_seq_len, max_q_len)]."""
        lib = _rq_lib.load()
        budget = _shared_workspace(device, "prefill", 0).numel()
        cap = max_blocks * BS
        groups, start, mx, mq = [], b0, 0, 0
        for b in range(b0, len(lens)):
            L = min(max(lens[b], 1), cap)
            n_mx, n_mq = max(mx, L), max(mq, q_lens[b])
            if b > start and lib.rq_int8_prefill_workspace_bytes(b + 1 - start, self.num_kv_heads, n_mx) > budget:
                groups.append((start, b, mx, mq))
                start, n_mx, n_mq = b, L, q_lens[b]
            mx, mq = n_mx, n_mq
        if start < len(lens):
            groups.append((start, len(lens), mx, mq))
        return groups

    def _fused_batch(self, query, kv_cache, md, output, num_actual_tokens):
        """A batch with multi-token sequences through the fused kernels: the leading
        single-token sequences (vLLM orders decodes first) go to the fused decode,
        the rest to the int8 prefill in groups that fit its workspace.  A prefill hook
        with the reference's signature (one sequence per call, no cu_seqlens_q:
        fused_paged_rq_int8_prefill.py:247-260, :305-309) is called once per sequence
        with that sequence's own query and output rows."""
        qsl_cpu = getattr(md, "rq_query_start_loc_cpu", None)
        sl_cpu = getattr(md, "rq_seq_lens_cpu", None)
        qsl_cpu = (qsl_cpu if qsl_cpu is not None else md.query_start_loc.cpu()).tolist()
        lens = (sl_cpu if sl_cpu is not None else md.seq_lens.cpu()).tolist()
        B = len(lens)
        q_lens = [qsl_cpu[b + 1] - qsl_cpu[b] for b in range(B)]
        nd = 0
        if self._fused_paged_available:
            while nd < B and q_lens[nd] == 1:
                nd += 1
        if nd:
            self._fused_decode(query, kv_cache, md.block_table[:nd], md.seq_lens[:nd], output, nd)
        if nd == B:
            return output
        kc, vc, R = self._launch_operands()
        BS = kv_cache.shape[1]
        bt = md.block_table
        names = _accepted_keywords(_fused_paged_rq_int8_prefill_fn)
        if names is not None and "cu_seqlens_q" not in names:
            for b in range(nd, B):
                s0, s1 = qsl_cpu[b], qsl_cpu[b + 1]
                if s1 > s0:
                    _call_hook(_fused_paged_rq_int8_prefill_fn, query[s0:s1], kv_cache, bt[b:b + 1],
                               md.seq_lens[b:b + 1], kc, vc, R, self.num_kv_heads, self.head_size, BS,
                               sm_scale=self.scale, out=output[s0:s1], **self._layout_kw())
            return output
        for g0, g1, mx, mq in self._prefill_groups(lens, q_lens, nd, BS, bt.shape[1], query.device):
            _call_hook(_fused_paged_rq_int8_prefill_fn, query[:num_actual_tokens], kv_cache, bt[g0:g1],
                       md.seq_lens[g0:g1], kc, vc, R, self.num_kv_heads, self.head_size, BS, sm_scale=self.scale,
                       out=output[:num_actual_tokens], cu_seqlens_q=md.query_start_loc[g0:g1 + 1], max_q_len=mq,
                       max_seq_len=mx, **self._layout_kw())
        return output

    # -- non-fused path -----------------------------------------------------------

    def _unfused_kernel_ok(self, dtype, num_heads: int) -> bool:
        """The non-fused kernels take this layer's shapes and dtype."""
        return (_paged_attention_fn is not None and dtype in (torch.float16, torch.bfloat16)
                and _fused_shape_ok(num_heads, self.num_kv_heads, self.head_size) is None)

    def _forward_unfused(self, query, kv_cache, md, output, num_actual_tokens):
        """Non-fused path (replaces :937-1036: q pre-rotation, paged decompress to the q
        dtype, flash_attn_varlen_func, back-rotation).

        head_size 128, f16/bf16: a batch of single-token decodes takes the decode kernel
        (rq_fused_decode: its arithmetic is this path's -- K/V rounded to the q dtype,
        exact Q K^T products, fp32 sums -- and a decode sees its whole context, causal
        or not; the batch's tiles are split over the whole GPU, and the launch is
        capturable in a HIP graph).  Other queries of at most RQ_UNFUSED_SHORT_Q tokens
        take one rq_paged_attention launch (K/V tiles dequantized to the q dtype in
        LDS; no workspace, no host read of the metadata, capturable).  A batch with
        longer queries sends its leading single-token decodes (vLLM orders decodes
        first) to the decode kernel, the following short ones to rq_paged_attention
        and the rest to rq_paged_prefill (same arithmetic; each 64-key tile decoded
        once into the prefill workspace, in groups that fit it).  Other shapes: the
        device path _forward_unfused_torch."""
        q = query[:num_actual_tokens]
        if not self._unfused_kernel_ok(q.dtype, q.shape[1]):
            return self._forward_unfused_torch(query, kv_cache, md, output, num_actual_tokens)
        max_q = getattr(md, "max_query_len", None)
        qsl_cpu = None
        if max_q is None:
            qsl_cpu = getattr(md, "rq_query_start_loc_cpu", None)
            qsl_cpu = qsl_cpu if qsl_cpu is not None else md.query_start_loc.cpu()
            max_q = int((qsl_cpu[1:] - qsl_cpu[:-1]).max()) if qsl_cpu.numel() > 1 else 0
        decode_ok = _unfused_decode_fn is not None and _shared_workspace is not None
        if int(max_q) == 1 and decode_ok:
            self._fused_decode(query, kv_cache, md.block_table, md.seq_lens, output, num_actual_tokens,
                               fn=_unfused_decode_fn)
            return output
        kc, vc, R = self._launch_operands()
        BS = kv_cache.shape[1]
        causal = bool(getattr(md, "causal", True))
        out = output[:num_actual_tokens]
        if int(max_q) <= RQ_UNFUSED_SHORT_Q or _paged_prefill_fn is None or _shared_workspace is None:
            _paged_attention_fn(q, kv_cache, md.block_table, md.seq_lens, md.query_start_loc, int(max_q), kc, vc, R,
                                self.num_kv_heads, self.head_size, BS, sm_scale=self.scale, causal=causal, out=out,
                                **self._layout_kw())
            return output
        if qsl_cpu is None:
            qsl_cpu = getattr(md, "rq_query_start_loc_cpu", None)
            qsl_cpu = qsl_cpu if qsl_cpu is not None else md.query_start_loc.cpu()
        sl_cpu = getattr(md, "rq_seq_lens_cpu", None)
        qsl = qsl_cpu.tolist()
        lens = (sl_cpu if sl_cpu is not None else md.seq_lens.cpu()).tolist()
        B = len(lens)
        q_lens = [qsl[b + 1] - qsl[b] for b in range(B)]
        nd = 0
        if decode_ok:
            while nd < B and q_lens[nd] == 1:
                nd += 1
        bt = md.block_table
        if nd:
            self._fused_decode(query, kv_cache, bt[:nd], md.seq_lens[:nd], output, nd, fn=_unfused_decode_fn)
        ns = nd
        while ns < B and q_lens[ns] <= RQ_UNFUSED_SHORT_Q:
            ns += 1
        if ns > nd:
            _paged_attention_fn(q, kv_cache, bt[nd:ns], md.seq_lens[nd:ns], md.query_start_loc[nd:ns + 1],
                                max(q_lens[nd:ns]), kc, vc, R, self.num_kv_heads, self.head_size, BS,
                                sm_scale=self.scale, causal=causal, out=out, **self._layout_kw())
        for g0, g1, mx, mq in self._prefill_groups(lens, q_lens, ns, BS, bt.shape[1], query.device):
            _paged_prefill_fn(q, kv_cache, bt[g0:g1], md.seq_lens[g0:g1], md.query_start_loc[g0:g1 + 1], mq, kc, vc,
                              R, self.num_kv_heads, self.head_size, BS, sm_scale=self.scale, causal=causal, out=out,
                              max_seq_len=mx, **self._layout_kw())
        return output

    def _forward_unfused_torch(self, query, kv_cache, md, output, num_actual_tokens):
        """Paged decompress + fp32 attention on the device, for shapes rq_paged_attention
        does not take (head sizes other than 128, GQA groups above 16, fp32 models).

        K/V of the referenced blocks are decompressed once (rq_paged_decompress) to
        the q dtype, as the reference's _decompress_cache_paged(..., query.dtype)
        (reference rq_backend.py:988-994); each sequence attends over its blocks in
        fp32, one kv head (its GQA group of query heads) and at most ~32 M scores at
        a time.  Host lengths come from the metadata's host copies when present
        (one device read otherwise)."""
        if query.device.type == "cuda" and torch.cuda.is_current_stream_capturing():
            raise RuntimeError("RotorQuant: this layer's shape or dtype runs the torch fallback (a loop over host "
                               "sequence lengths), which cannot be captured in a graph")
        BS = kv_cache.shape[1]
        H, D = self.num_kv_heads, self.head_size
        q = query[:num_actual_tokens]
        HQ = q.shape[1]
        G = HQ // H
        causal = bool(getattr(md, "causal", True))
        q_rot = (q.float() @ self._dev_R.T).to(q.dtype).float()
        qsl = getattr(md, "rq_query_start_loc_cpu", None)
        if qsl is None:
            qsl = getattr(md, "query_start_loc", None)
            qsl = qsl.cpu() if qsl is not None else torch.tensor([0, num_actual_tokens])
        sl = getattr(md, "rq_seq_lens_cpu", None)
        lens = (sl if sl is not None else md.seq_lens.cpu()).tolist()
        starts = qsl.tolist()
        # capacity: every referenced block once (fewer when sequences share blocks)
        cap = max(1, sum((L + BS - 1) // BS for L in lens))
        out_k = torch.empty(cap, BS, H, D, dtype=q.dtype, device=q.device)
        k_cache, v_cache, bt, _ = _paged_decompress_fn(kv_cache, md.block_table, md.seq_lens, H, D, self._dev_kc,
                                                       self._dev_vc, q.dtype, out_k=out_k,
                                                       out_v=torch.empty_like(out_k), **self._layout_kw())
        out_rot = torch.zeros(num_actual_tokens, HQ, D, dtype=torch.float32, device=q.device)
        for b, L in enumerate(lens):
            s0, s1 = starts[b], starts[b + 1]
            T = s1 - s0
            if T <= 0 or L == 0:
                continue
            ids = bt[b, :(L + BS - 1) // BS].long()
            K = k_cache[ids].reshape(-1, H, D)[:L].float()
            V = v_cache[ids].reshape(-1, H, D)[:L].float()
            rows = max(1, min(T, (32 << 20) // max(1, G * L)))
            for r0 in range(0, T, rows):
                r1 = min(T, r0 + rows)
                pos = (L - T + r0) + torch.arange(r1 - r0, device=q.device)
                if not causal:
                    pos = torch.full_like(pos, L - 1)
                masked = torch.arange(L, device=q.device)[None, :] > pos[:, None]  # (rows, L)
                for h in range(H):
                    Qh = q_rot[s0 + r0:s0 + r1, h * G:(h + 1) * G, :].reshape(-1, D)  # (rows*G, D)
                    S = (Qh @ K[:, h, :].T) * self.scale  # (rows*G, L)
                    S = S.view(r1 - r0, G, L).masked_fill_(masked[:, None, :], float("-inf"))
                    P = torch.softmax(S, dim=-1).view(-1, L)
                    out_rot[s0 + r0:s0 + r1, h * G:(h + 1) * G, :] = (P @ V[:, h, :]).view(r1 - r0, G, D)
        out_rot = out_rot.to(q.dtype).float()
        output[:num_actual_tokens] = (out_rot @ self._dev_R).to(output.dtype)
        return output

    # -- forward -------------------------------------------------------------

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None, output_scale=None,
                output_block_scale=None):
        """compress/store new K/V, then attention from the packed cache (reference :858-1036).

        Dispatch: a batch of single-token decodes -> fused decode (graph-capturable);
        one multi-token sequence -> the int8 prefill with the reference's arguments;
        a batch with several sequences and multi-token ones -> leading decodes to
        the fused decode, the rest to the int8 prefill; without RQ_USE_FUSED_PAGED
        (or for shapes the fused kernels do not take) -> the non-fused path
        (_forward_unfused)."""
        assert output is not None, "Output tensor must be provided."
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("Fused output quantization is not supported with RotorQuant backend")
        if attn_metadata is None or kv_cache is None:
            return output.zero_()
        if self.attn_type in (AttentionType.ENCODER_ONLY, AttentionType.ENCODER):
            n = attn_metadata.num_actual_tokens
            return self._forward_encoder_attention(query[:n], key[:n], value[:n], output[:n], attn_metadata, layer)

        num_actual_tokens = attn_metadata.num_actual_tokens
        max_query_len = getattr(attn_metadata, "max_query_len", None)
        # A single token (reference :904), or a uniform batch of single-token decodes.
        is_decode = num_actual_tokens == 1 or max_query_len == 1
        if not self._cg_buffers_ready:
            self._init_cg_buffers(kv_cache, query.dtype)
        if key is not None and value is not None:
            self._compress_and_store(key, value, kv_cache, attn_metadata.slot_mapping)

        if is_decode and self._fused_paged_available:
            self._fused_decode(query, kv_cache, attn_metadata.block_table, attn_metadata.seq_lens, output,
                               num_actual_tokens)
            return output

        use_cascade = getattr(attn_metadata, "use_cascade", False)
        if not is_decode and self._fused_prefill_available and not use_cascade:
            if attn_metadata.seq_lens.numel() == 1:
                # the reference's call (fused_paged_rq_int8_prefill.py:247-260), plus this
                # build's workspace when the hook takes it
                kc, vc, R = self._launch_operands()
                _call_hook(_fused_paged_rq_int8_prefill_fn, query[:num_actual_tokens], kv_cache,
                           attn_metadata.block_table, attn_metadata.seq_lens, kc, vc, R, self.num_kv_heads,
                           self.head_size, kv_cache.shape[1], sm_scale=self.scale, out=output[:num_actual_tokens],
                           **self._layout_kw())
                return output
            return self._fused_batch(query, kv_cache, attn_metadata, output, num_actual_tokens)

        if use_cascade:
            raise NotImplementedError("RQ does not yet support cascade attention")
        return self._forward_unfused(query, kv_cache, attn_metadata, output, num_actual_tokens)


# ---------------------------------------------------------------------------
# Registration (reference: rq_backend.py:1043-1093)
# ---------------------------------------------------------------------------

_original_get_kv_cache_spec = None


def register_rq_backend() -> None:
    """Register RotorQuant as vLLM's CUSTOM attention backend and make decoder
    attention layers report RQFullAttentionSpec (uint8 pages sized for the packed slots)."""
    global _original_get_kv_cache_spec
    from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend

    register_backend(AttentionBackendEnum.CUSTOM, "rotorquant_vllm.vllm.rq_backend.RQAttentionBackend")

    from vllm.v1.core.single_type_kv_cache_manager import spec_manager_map

    if RQFullAttentionSpec not in spec_manager_map:
        spec_manager_map[RQFullAttentionSpec] = spec_manager_map[FullAttentionSpec]

    from vllm.model_executor.layers.attention.attention import Attention

    if _original_get_kv_cache_spec is None:
        _original_get_kv_cache_spec = Attention.get_kv_cache_spec
    original = _original_get_kv_cache_spec

    def _rq_get_kv_cache_spec(self, vllm_config):
        spec = original(self, vllm_config)
        if isinstance(spec, FullAttentionSpec) and not isinstance(spec, RQFullAttentionSpec):
            kwargs = {f.name: getattr(spec, f.name) for f in dc_fields(spec)}
            kwargs["dtype"] = torch.uint8
            return RQFullAttentionSpec(**kwargs)
        return spec

    Attention.get_kv_cache_spec = _rq_get_kv_cache_spec
    logger.info("RQ attention backend registered as CUSTOM (compressed cache)")


__all__ = ["RQAttentionBackend", "RQAttentionImpl", "RQMetadataBuilder", "RQFullAttentionSpec",
           "register_rq_backend"]
