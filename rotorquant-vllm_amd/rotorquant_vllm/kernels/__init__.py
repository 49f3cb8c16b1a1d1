"""Op-level API of the gfx950 RotorQuant kernels.

Same names, signatures and argument meaning as the reference's op exports
(src/rotorquant_vllm/triton/__init__.py:1-15), backed by librq_hip.so through
the C ABI (include/rq_abi.h).  Differences, all deliberate:

* Inputs must be ROCm device tensors.  The reference silently takes a torch CPU
  path when `not x.is_cuda` (isoquant_compress.py:128-129); here a CPU tensor
  raises, so no result can come from anything but the HIP kernels.
* compress reads only the diagonal blocks of R^T (2x2, 4x4 or 8x8; checked
  once per rotation tensor) instead of a dense tiled product.
* fused_paged_rq_int8_prefill accepts any number of sequences (the reference
  raises ValueError for more than one, fused_paged_rq_int8_prefill.py:305-309)
  through the keyword `cu_seqlens_q`; with one sequence and no keyword it
  behaves as the reference: all q tokens are the sequence's last q_len tokens.
* paged_attention has no op-level counterpart: it is the backend's non-fused
  path (paged decompress + flash_attn_varlen_func + the two rotations,
  rq_backend.py:937-1036) as one launch; paged_prefill is the same arithmetic
  in two launches (each 64-key tile decoded once), for long queries.
"""
from __future__ import annotations

import math
import weakref

import torch

from .. import _lib

__all__ = [
    "iso_compress",
    "iso_decompress",
    "planar_compress",
    "planar_decompress",
    "fused_paged_rq_int8_prefill",
    "fused_paged_rq_decode",
    "compress_store",
    "paged_decompress",
    "paged_attention",
    "paged_prefill",
    "rotation_block",
    "shared_workspace",
]


def _require_device(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "rotorquant_vllm.kernels runs only on ROCm device tensors (got a "
                f"{t.device.type} tensor); there is no CPU path")
        dev = t.device if dev is None else dev
    _lib.load()
    return dev


# ---------------------------------------------------------------------------
# Rotation block structure (checked once per tensor)
# ---------------------------------------------------------------------------

# Keyed by tensor identity and checked against a weak reference to the tensor (a
# new tensor that reuses a freed tensor's memory, or even its id, never sees the
# old entry; entries are dropped when their tensor dies), with the tensor's
# version counter to catch in-place writes.
_block_cache: dict = {}


def _cache_get(t: torch.Tensor):
    ent = _block_cache.get(id(t))
    return ent if ent is not None and ent[0]() is t and ent[1] == t._version else None


def _cache_put(t: torch.Tensor, *vals):
    key = id(t)
    ref = weakref.ref(t, lambda _r, k=key: _block_cache.pop(k, None) if _block_cache.get(k, (None,))[0] is _r else None)
    _block_cache[key] = (ref, t._version, *vals)


def _block_of(RT: torch.Tensor) -> int:
    """Smallest width in (2, 4, 8) for which RT is block diagonal."""
    D = RT.shape[0]
    idx = torch.arange(D)
    for blk in (2, 4, 8):
        if D % blk:
            continue
        off = (idx[:, None] // blk) != (idx[None, :] // blk)
        if not bool((RT[off] != 0).any()):
            return blk
    raise ValueError("rotation is not block diagonal with 2x2, 4x4 or 8x8 blocks; "
                     "the HIP compress kernels read only the diagonal blocks")


def rotation_block(rotation: torch.Tensor) -> int:
    """Diagonal block width of a (D, D) rotation R (checked once per tensor and version)."""
    ent = _cache_get(rotation)
    if ent is None:
        _cache_put(rotation, _block_of(rotation.detach().float().cpu()))
        ent = _cache_get(rotation)
    return ent[2]


def _rt_block(rot_T_even: torch.Tensor, rot_T_odd: torch.Tensor) -> int:
    ent = _cache_get(rot_T_even)
    if ent is None or ent[3]() is not rot_T_odd or ent[4] != rot_T_odd._version:
        e, o = rot_T_even.detach().float().cpu(), rot_T_odd.detach().float().cpu()
        D = e.shape[0]
        RT = torch.empty(D, D)
        RT[:, 0::2] = e
        RT[:, 1::2] = o
        _cache_put(rot_T_even, _block_of(RT), weakref.ref(rot_T_odd), rot_T_odd._version)
        ent = _cache_get(rot_T_even)
    return ent[2]


def _f32(t: torch.Tensor, device) -> torch.Tensor:
    return t.to(device=device, dtype=torch.float32).contiguous()


def _layout(dense3: bool) -> int:
    """index_layout argument of the C ABI: RQ_INDEX_NIBBLE (0) or RQ_INDEX_DENSE3 (1)."""
    return 1 if dense3 else 0


# ---------------------------------------------------------------------------
# Compress / decompress
# ---------------------------------------------------------------------------

def _compress(x, rot_T_even, rot_T_odd, boundaries):
    dev = _require_device(x)
    N, H, D = x.shape
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"x must be fp16, bf16 or fp32, got {x.dtype}")
    blk = _rt_block(rot_T_even, rot_T_odd)
    x_flat = x.reshape(N * H, D).contiguous()
    re, ro, b = _f32(rot_T_even, dev), _f32(rot_T_odd, dev), _f32(boundaries, dev)
    packed = torch.empty(N, H, D // 2, dtype=torch.uint8, device=dev)
    norms = torch.empty(N, H, 1, dtype=torch.float32, device=dev)
    rc = _lib.load().rq_compress(x_flat.data_ptr(), _lib.dtype_code(x.dtype), N * H, D, re.data_ptr(),
                                 ro.data_ptr(), blk, b.data_ptr(), b.numel(), packed.data_ptr(),
                                 norms.data_ptr(), _lib.stream_ptr(dev))
    _lib.check(rc, "rq_compress")
    return packed, norms


def iso_compress(x: torch.Tensor, rot_T_even: torch.Tensor, rot_T_odd: torch.Tensor,
                 boundaries: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(N, H, D) fp16/bf16 -> nibble-packed (N, H, D/2) uint8 + (N, H, 1) fp32 norms.

    Reference: src/rotorquant_vllm/triton/isoquant_compress.py:104-158.
    """
    return _compress(x, rot_T_even, rot_T_odd, boundaries)


def planar_compress(x: torch.Tensor, rot_T_even: torch.Tensor, rot_T_odd: torch.Tensor,
                    boundaries: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """PlanarQuant compress; reference: src/rotorquant_vllm/triton/planarquant_compress.py:100-154."""
    return _compress(x, rot_T_even, rot_T_odd, boundaries)


def _decompress(packed, norms, centroids, dtype):
    dev = _require_device(packed, norms)
    N, H, half = packed.shape
    D = 2 * half
    p = packed.reshape(N * H, half).contiguous()
    n = norms.reshape(N * H).to(torch.float32).contiguous()
    c = _f32(centroids, dev)
    out = torch.empty(N, H, D, dtype=dtype, device=dev)
    rc = _lib.load().rq_decompress(p.data_ptr(), n.data_ptr(), N * H, D, c.data_ptr(), c.numel(),
                                   out.data_ptr(), _lib.dtype_code(dtype), _lib.stream_ptr(dev))
    _lib.check(rc, "rq_decompress")
    return out


def iso_decompress(packed: torch.Tensor, norms: torch.Tensor, centroids: torch.Tensor,
                   dtype: torch.dtype) -> torch.Tensor:
    """(N, H, D/2) uint8 + (N, H, 1) fp32 -> (N, H, D) rotated-space values.

    Reference: src/rotorquant_vllm/triton/isoquant_decompress.py:63-100.
    """
    return _decompress(packed, norms, centroids, dtype)


def planar_decompress(packed: torch.Tensor, norms: torch.Tensor, centroids: torch.Tensor,
                      dtype: torch.dtype) -> torch.Tensor:
    """Reference: src/rotorquant_vllm/triton/planarquant_decompress.py:63-101."""
    return _decompress(packed, norms, centroids, dtype)


# ---------------------------------------------------------------------------
# Fused K+V compress into the paged cache
# ---------------------------------------------------------------------------

def compress_store(key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor, slot_mapping: torch.Tensor,
                   rot_T_even: torch.Tensor, rot_T_odd: torch.Tensor, k_boundaries: torch.Tensor,
                   v_boundaries: torch.Tensor, rot_block: int | None = None, dense3: bool = False) -> None:
    """Compress key/value (N, H, D) and write full slots of kv_cache (NB, BS, total_bytes).

    Replaces RQAttentionImpl._compress_and_store (rq_backend.py:585-657).
    Slots < 0 are skipped.  dense3: write the dense 3-bit index layout
    (RQ_INDEX_DENSE3 in include/rq_abi.h; 3-bit codebooks only).
    """
    dev = _require_device(key, value, kv_cache, slot_mapping)
    N, H, D = key.shape
    if value.shape != key.shape or value.dtype != key.dtype:
        raise ValueError("key and value must have the same shape and dtype")
    if key.stride(-1) != 1 or value.stride(-1) != 1:
        raise ValueError("key/value must be contiguous over head_dim")
    if kv_cache.dtype != torch.uint8 or kv_cache.dim() != 3:
        raise ValueError("kv_cache must be a (num_blocks, block_size, total_bytes) uint8 tensor")
    blk = rot_block if rot_block is not None else _rt_block(rot_T_even, rot_T_odd)
    sm = slot_mapping.to(torch.int64).contiguous()
    if sm.numel() < N:
        raise ValueError("slot_mapping shorter than the number of tokens")
    N = min(N, sm.numel())
    NB, BS, TB = kv_cache.shape
    kb, vb = _f32(k_boundaries, dev), _f32(v_boundaries, dev)
    rc = _lib.load().rq_compress_store(
        key.data_ptr(), value.data_ptr(), _lib.dtype_code(key.dtype), N, key.stride(0), key.stride(1),
        value.stride(0), value.stride(1), H, D, _layout(dense3), sm.data_ptr(), kv_cache.data_ptr(), NB, BS,
        kv_cache.stride(0), kv_cache.stride(1), TB, _f32(rot_T_even, dev).data_ptr(),
        _f32(rot_T_odd, dev).data_ptr(), blk, kb.data_ptr(), kb.numel(), vb.data_ptr(), vb.numel(),
        _lib.stream_ptr(dev))
    _lib.check(rc, "rq_compress_store")


# ---------------------------------------------------------------------------
# Paged decompress (non-fused path)
# ---------------------------------------------------------------------------

def paged_decompress(kv_cache: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor,
                     num_kv_heads: int, head_dim: int, k_centroids: torch.Tensor, v_centroids: torch.Tensor,
                     dtype: torch.dtype, out_k: torch.Tensor | None = None, out_v: torch.Tensor | None = None,
                     workspace: torch.Tensor | None = None, dense3: bool = False):
    """Decompress the physical blocks referenced by block_table.

    Returns (key_cache, value_cache, remapped_block_table, num_unique) with
    key/value of shape (capacity, BS, H, D); the first num_unique blocks hold
    the referenced physical blocks in ascending physical order, as the
    reference's _decompress_cache_paged (rq_backend.py:737-852).  num_unique is
    a 1-element device int32 tensor (no host sync).  dense3: the cache holds the
    dense 3-bit index layout.
    """
    dev = _require_device(kv_cache, block_table, seq_lens)
    NB, BS, _ = kv_cache.shape
    bt = block_table.to(torch.int32)
    if bt.stride(-1) != 1:
        bt = bt.contiguous()
    sl = seq_lens.to(torch.int32).contiguous()
    B, MB = bt.shape
    cap = NB if out_k is None else out_k.shape[0]
    if out_k is None:
        out_k = torch.empty(cap, BS, num_kv_heads, head_dim, dtype=dtype, device=dev)
    if out_v is None:
        out_v = torch.empty_like(out_k)
    need = _lib.load().rq_paged_decompress_workspace_bytes(NB)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    remapped = torch.empty(B, MB, dtype=torch.int32, device=dev)
    count = torch.empty(1, dtype=torch.int32, device=dev)
    kc, vc = _f32(k_centroids, dev), _f32(v_centroids, dev)
    rc = _lib.load().rq_paged_decompress(
        kv_cache.data_ptr(), NB, BS, kv_cache.stride(0), kv_cache.stride(1), num_kv_heads, head_dim,
        _layout(dense3), bt.data_ptr(), B, MB, bt.stride(0), sl.data_ptr(), kc.data_ptr(), kc.numel(), vc.data_ptr(),
        vc.numel(), out_k.data_ptr(), out_v.data_ptr(), _lib.dtype_code(dtype), cap, remapped.data_ptr(),
        count.data_ptr(), workspace.data_ptr(), workspace.numel(), _lib.stream_ptr(dev))
    _lib.check(rc, "rq_paged_decompress")
    return out_k, out_v, remapped, count


# ---------------------------------------------------------------------------
# Fused paged decode
# ---------------------------------------------------------------------------

_ws_cache: dict = {}
_ws_retired: list = []


def shared_workspace(device, kind: str, nbytes: int) -> torch.Tensor:
    """Device scratch of one kind per device ("decode": split-KV partials, query
    operands, tile descriptors; "prefill": int8 tile images), shared by every call
    on the device's stream (calls run one after another; every call rewrites what
    it reads).  When a call needs more, a larger buffer replaces it and the old one
    is kept allocated until the process ends, so a HIP graph that captured its
    address never sees it freed and reused."""
    key = (str(device), kind)
    buf = _ws_cache.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _ws_retired.append(buf)
        buf = torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)
        _ws_cache[key] = buf
    return buf


def _fused_decode_call(q, kv_cache, block_table, seq_lens, centroids_k, centroids_v, rotation, num_kv_heads,
                       head_dim, block_size, sm_scale, out, max_seq_len, workspace, dense3=False):
    """Validated argument tuple of one rq_fused_decode call (tensors it creates are returned to keep them alive)."""
    num_seqs, H_Q, D = q.shape
    assert D == head_dim, f"D={D} != head_dim={head_dim}"
    assert H_Q % num_kv_heads == 0
    assert kv_cache.dtype == torch.uint8
    assert block_table.dtype == torch.int32
    assert seq_lens.dtype == torch.int32
    dev = _require_device(q, kv_cache, block_table, seq_lens)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(head_dim)
    if q.stride(-1) != 1:
        q = q.contiguous()
    if out is None:
        out = torch.empty_like(q)
    if block_table.stride(-1) != 1:
        block_table = block_table.contiguous()
    MB = block_table.shape[1]
    if max_seq_len is None:
        max_seq_len = MB * block_size
    blk = rotation_block(rotation)
    L = _lib.load()
    need = L.rq_fused_decode_workspace_bytes(num_seqs, H_Q, head_dim, max_seq_len)
    ws = workspace if workspace is not None and workspace.numel() >= need else shared_workspace(dev, "decode", need)
    R = _f32(rotation, dev)
    kc, vc = _f32(centroids_k, dev), _f32(centroids_v, dev)
    sl = seq_lens.contiguous()
    args = (q.data_ptr(), _lib.dtype_code(q.dtype), num_seqs, H_Q, q.stride(0), q.stride(1), kv_cache.data_ptr(),
            kv_cache.shape[0], block_size, kv_cache.stride(0), kv_cache.stride(1), num_kv_heads, head_dim,
            _layout(dense3), block_table.data_ptr(), MB, block_table.stride(0), sl.data_ptr(), max_seq_len,
            kc.data_ptr(), kc.numel(),
            vc.data_ptr(), vc.numel(), R.data_ptr(), blk, float(sm_scale), out.data_ptr(), out.stride(0),
            out.stride(1), ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
    return L, args, out, (q, block_table, R, kc, vc, sl, ws)


def fused_paged_rq_decode(q: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor,
                          seq_lens: torch.Tensor, centroids_k: torch.Tensor, centroids_v: torch.Tensor,
                          rotation: torch.Tensor, num_kv_heads: int, head_dim: int, block_size: int,
                          sm_scale: float | None = None, out: torch.Tensor | None = None,
                          max_seq_len: int | None = None, workspace: torch.Tensor | None = None,
                          dense3: bool = False) -> torch.Tensor:
    """Fused paged decode attention; q (num_seqs, H_Q, D) in original space -> output in original space.

    Reference: src/rotorquant_vllm/triton/fused_paged_rq_decode.py:214-312 (same
    arguments; `max_seq_len` optionally bounds seq_lens and sizes the split-KV
    grid, default block_table.shape[1] * block_size; `workspace` optionally
    supplies the scratch, a uint8 device tensor of at least
    rq_fused_decode_workspace_bytes(...) bytes, reusable across calls; dense3:
    the cache holds the dense 3-bit index layout).
    """
    L, args, out, _keep = _fused_decode_call(q, kv_cache, block_table, seq_lens, centroids_k, centroids_v, rotation,
                                             num_kv_heads, head_dim, block_size, sm_scale, out, max_seq_len, workspace,
                                             dense3)
    _lib.check(L.rq_fused_decode(*args), "rq_fused_decode")
    return out


def fused_paged_rq_decode_launcher(q: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor,
                                   seq_lens: torch.Tensor, centroids_k: torch.Tensor, centroids_v: torch.Tensor,
                                   rotation: torch.Tensor, num_kv_heads: int, head_dim: int, block_size: int,
                                   sm_scale: float | None = None, out: torch.Tensor | None = None,
                                   max_seq_len: int | None = None, workspace: torch.Tensor | None = None,
                                   dense3: bool = False, kernel_events=None):
    """Validate once and return a zero-argument callable that re-issues the same
    rq_fused_decode call (same buffers, the stream current now) without
    per-call Python work -- for loops over static buffers such as a benchmark.
    The callable returns `out`; the tensors must outlive it.

    kernel_events: optional (start, stop) torch.cuda.Event pair (enable_timing=True)
    recorded at the start and the end of the call's decode kernel alone
    (rq_fused_decode_timed), for measuring that kernel's own duration."""
    L, args, out, keep = _fused_decode_call(q, kv_cache, block_table, seq_lens, centroids_k, centroids_v, rotation,
                                            num_kv_heads, head_dim, block_size, sm_scale, out, max_seq_len, workspace,
                                            dense3)
    fn, name = L.rq_fused_decode, "rq_fused_decode"
    if kernel_events is not None:
        for ev in kernel_events:
            if not ev.cuda_event:  # torch creates the HIP event at its first record
                ev.record()
        args = args + tuple(ev._as_parameter_ for ev in kernel_events)
        fn, name = L.rq_fused_decode_timed, "rq_fused_decode_timed"
        keep = keep + tuple(kernel_events)

    def launch():
        rc = fn(*args)
        if rc:
            _lib.check(rc, name)
        return out

    launch.keep = keep
    return launch


# ---------------------------------------------------------------------------
# INT8 prefill
# ---------------------------------------------------------------------------

def _single_cu_seqlens(device, num_tokens: int) -> torch.Tensor:
    """[0, num_tokens] made on the device by a fill kernel: the reference's
    single-sequence call form then costs no host-to-device copy per call and stays
    capturable in a HIP graph."""
    return torch.arange(2, dtype=torch.int32, device=device).mul_(int(num_tokens))


def fused_paged_rq_int8_prefill(q: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor,
                                seq_lens: torch.Tensor, k_centroids: torch.Tensor, v_centroids: torch.Tensor,
                                rotation: torch.Tensor, num_kv_heads: int, head_dim: int, block_size: int,
                                sm_scale: float | None = None, out: torch.Tensor | None = None,
                                cu_seqlens_q: torch.Tensor | None = None,
                                max_q_len: int | None = None, max_seq_len: int | None = None,
                                workspace: torch.Tensor | None = None, dense3: bool = False) -> torch.Tensor:
    """Causal prefill attention from the packed cache with Q K^T and P V on int8 MFMA.

    Reference: src/rotorquant_vllm/triton/fused_paged_rq_int8_prefill.py:247-363.
    q: (num_tokens, H_Q, D); block_table (num_seqs, max_blocks) int32; seq_lens
    (num_seqs,) int32 total context lengths (new tokens included).
    cu_seqlens_q (num_seqs + 1,) int32 splits q among sequences; without it
    there must be one sequence (as in the reference).
    max_seq_len bounds every seq_lens entry (default: the block table's capacity)
    and sizes the int8 tile-image workspace; workspace may be passed to reuse a
    buffer of rq_int8_prefill_workspace_bytes bytes.  dense3: the cache holds the
    dense 3-bit index layout.
    """
    num_tokens, H_Q, D = q.shape
    assert D == head_dim
    assert H_Q % num_kv_heads == 0
    assert kv_cache.dtype == torch.uint8
    assert block_table.dtype == torch.int32
    assert seq_lens.dtype == torch.int32
    if cu_seqlens_q is None:
        if seq_lens.numel() != 1:
            raise ValueError(
                f"fused_paged_rq_int8_prefill supports only a single sequence, "
                f"but got seq_lens.numel() == {seq_lens.numel()}.")
        cu_seqlens_q = _single_cu_seqlens(q.device, num_tokens)
        max_q_len = num_tokens
    dev = _require_device(q, kv_cache, block_table, seq_lens, cu_seqlens_q)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(head_dim)
    if q.stride(-1) != 1:
        q = q.contiguous()
    if out is None:
        out = torch.empty_like(q)
    bt = block_table if block_table.dim() == 2 else block_table.reshape(1, -1)
    if bt.stride(-1) != 1:
        bt = bt.contiguous()
    num_seqs = seq_lens.numel()
    if max_q_len is None:
        max_q_len = num_tokens
    blk = rotation_block(rotation)
    R = _f32(rotation, dev)
    kc, vc = _f32(k_centroids, dev), _f32(v_centroids, dev)
    cu = cu_seqlens_q.to(torch.int32).contiguous()
    if max_seq_len is None:
        max_seq_len = bt.shape[1] * block_size
    L = _lib.load()
    need = L.rq_int8_prefill_workspace_bytes(num_seqs, num_kv_heads, max_seq_len)
    ws = workspace if workspace is not None and workspace.numel() >= need else shared_workspace(dev, "prefill", need)
    rc = L.rq_int8_prefill(
        q.data_ptr(), _lib.dtype_code(q.dtype), num_tokens, H_Q, q.stride(0), q.stride(1), cu.data_ptr(),
        num_seqs, max_q_len, kv_cache.data_ptr(), kv_cache.shape[0], block_size, kv_cache.stride(0),
        kv_cache.stride(1), num_kv_heads, head_dim, _layout(dense3), bt.data_ptr(), bt.shape[1], bt.stride(0),
        seq_lens.contiguous().data_ptr(), max_seq_len, kc.data_ptr(), kc.numel(), vc.data_ptr(), vc.numel(),
        R.data_ptr(), blk, float(sm_scale), out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(), ws.numel(),
        _lib.stream_ptr(dev))
    _lib.check(rc, "rq_int8_prefill")
    return out


# ---------------------------------------------------------------------------
# Non-fused path: attention over K/V dequantized to the q dtype in-kernel
# ---------------------------------------------------------------------------

def paged_attention(q: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor,
                    cu_seqlens_q: torch.Tensor, max_q_len: int, k_centroids: torch.Tensor,
                    v_centroids: torch.Tensor, rotation: torch.Tensor, num_kv_heads: int, head_dim: int,
                    block_size: int, sm_scale: float | None = None, causal: bool = True,
                    out: torch.Tensor | None = None, dense3: bool = False) -> torch.Tensor:
    """Attention of the new query tokens over the packed cache, q and output in original space.

    The reference's non-fused path (rq_backend.py:937-1036: q_rot = q R^T cast to
    q's dtype, paged decompress to q's dtype, flash_attn_varlen_func, out_rot R)
    as one kernel that dequantizes K/V tiles into LDS (rq_paged_attention).
    q: (num_tokens, H_Q, D); cu_seqlens_q (num_seqs + 1,) int32; seq_lens
    (num_seqs,) int32 context lengths including the new tokens; max_q_len: a host
    int bounding every q_len (it sizes the grid).  Query i of sequence b sits at
    position seq_lens[b] - q_len_b + i.  dense3: the cache holds the dense 3-bit
    index layout.
    """
    num_tokens, H_Q, D = q.shape
    assert D == head_dim
    assert H_Q % num_kv_heads == 0
    assert kv_cache.dtype == torch.uint8
    assert block_table.dtype == torch.int32 and seq_lens.dtype == torch.int32
    assert cu_seqlens_q.dtype == torch.int32
    dev = _require_device(q, kv_cache, block_table, seq_lens, cu_seqlens_q)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(head_dim)
    if q.stride(-1) != 1:
        q = q.contiguous()
    if out is None:
        out = torch.empty_like(q)
    bt = block_table if block_table.stride(-1) == 1 else block_table.contiguous()
    blk = rotation_block(rotation)
    R = _f32(rotation, dev)
    kc, vc = _f32(k_centroids, dev), _f32(v_centroids, dev)
    cu, sl = cu_seqlens_q.contiguous(), seq_lens.contiguous()
    L = _lib.load()
    rc = L.rq_paged_attention(
        q.data_ptr(), _lib.dtype_code(q.dtype), num_tokens, H_Q, q.stride(0), q.stride(1), cu.data_ptr(),
        sl.numel(), int(max_q_len), 1 if causal else 0, kv_cache.data_ptr(), kv_cache.shape[0], block_size,
        kv_cache.stride(0), kv_cache.stride(1), num_kv_heads, head_dim, _layout(dense3), bt.data_ptr(), bt.shape[1],
        bt.stride(0),
        sl.data_ptr(), kc.data_ptr(), kc.numel(), vc.data_ptr(), vc.numel(), R.data_ptr(), blk, float(sm_scale),
        out.data_ptr(), out.stride(0), out.stride(1), _lib.stream_ptr(dev))
    _lib.check(rc, "rq_paged_attention")
    return out


def paged_prefill(q: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor,
                  cu_seqlens_q: torch.Tensor, max_q_len: int, k_centroids: torch.Tensor, v_centroids: torch.Tensor,
                  rotation: torch.Tensor, num_kv_heads: int, head_dim: int, block_size: int,
                  sm_scale: float | None = None, causal: bool = True, out: torch.Tensor | None = None,
                  max_seq_len: int | None = None, workspace: torch.Tensor | None = None,
                  dense3: bool = False) -> torch.Tensor:
    """paged_attention's arithmetic (the reference's non-fused path, rq_backend.py:937-1036)
    in two launches for long queries (rq_paged_prefill): every 64-key tile of every
    (sequence, kv head) is decoded once into a tile image (K and V in q's dtype),
    then streamed by the attention kernel.

    Arguments as for paged_attention; max_seq_len bounds every seq_lens entry
    (default: the block table's capacity) and sizes the workspace, which may be
    passed (rq_paged_prefill_workspace_bytes bytes) or comes from the shared
    per-device prefill buffer.
    """
    num_tokens, H_Q, D = q.shape
    assert D == head_dim
    assert H_Q % num_kv_heads == 0
    assert kv_cache.dtype == torch.uint8
    assert block_table.dtype == torch.int32 and seq_lens.dtype == torch.int32
    assert cu_seqlens_q.dtype == torch.int32
    dev = _require_device(q, kv_cache, block_table, seq_lens, cu_seqlens_q)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(head_dim)
    if q.stride(-1) != 1:
        q = q.contiguous()
    if out is None:
        out = torch.empty_like(q)
    bt = block_table if block_table.stride(-1) == 1 else block_table.contiguous()
    blk = rotation_block(rotation)
    R = _f32(rotation, dev)
    kc, vc = _f32(k_centroids, dev), _f32(v_centroids, dev)
    cu, sl = cu_seqlens_q.contiguous(), seq_lens.contiguous()
    if max_seq_len is None:
        max_seq_len = bt.shape[1] * block_size
    L = _lib.load()
    need = L.rq_paged_prefill_workspace_bytes(sl.numel(), num_kv_heads, max_seq_len)
    ws = workspace if workspace is not None and workspace.numel() >= need else shared_workspace(dev, "prefill", need)
    rc = L.rq_paged_prefill(
        q.data_ptr(), _lib.dtype_code(q.dtype), num_tokens, H_Q, q.stride(0), q.stride(1), cu.data_ptr(),
        sl.numel(), int(max_q_len), 1 if causal else 0, kv_cache.data_ptr(), kv_cache.shape[0], block_size,
        kv_cache.stride(0), kv_cache.stride(1), num_kv_heads, head_dim, _layout(dense3), bt.data_ptr(), bt.shape[1],
        bt.stride(0), sl.data_ptr(), max_seq_len, kc.data_ptr(), kc.numel(), vc.data_ptr(), vc.numel(), R.data_ptr(),
        blk, float(sm_scale), out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(), ws.numel(),
        _lib.stream_ptr(dev))
    _lib.check(rc, "rq_paged_prefill")
    return out
