"""TEST INFRASTRUCTURE ONLY -- CPU oracle for the RotorQuant KV-cache hot path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker.  The product (rotorquant-vllm_amd/) never
calls it.

Restates the reference (tpurtell/rotorquant-vllm) on the CPU:

  compress / decompress ........ rq_oracle.c (bit-exact restatement, see there);
                                 reference_cpu_compress / _decompress: the same
                                 torch CPU op sequence, timed as bench.py's CPU baseline
  lloyd_max_closed_form ........ src/rotorquant_vllm/quantization/lloyd_max.py:32-86
                                 (same schedule, exact Gaussian integrals)
  slot layout .................. src/rotorquant_vllm/vllm/rq_backend.py:155-188, :482-490
  dense3_pack / _unpack ........ the opt-in dense 3-bit index layout (this build's own
                                 format; the reference only lists it on its roadmap,
                                 PKG-INFO:110)
  compress_store ............... rq_backend.py:585-657
  paged_decompress ............. rq_backend.py:737-852
  decode_attention ............. src/rotorquant_vllm/triton/fused_paged_rq_decode.py:252-312
                                 (math of the kernel :76-206 in fp64; K and V are
                                 centroid * norm rounded to the q dtype, :146-147, :190-191)
  prefill_attention ............ src/rotorquant_vllm/triton/fused_paged_rq_int8_prefill.py:296-363
                                 (math in fp64; K and V rounded to the q dtype, :172, :224;
                                 causal position offset L - T + i)
  unfused_attention ............ src/rotorquant_vllm/vllm/rq_backend.py:937-1036 (the
                                 non-fused path: K/V decompressed to the q dtype,
                                 flash attention's math in fp64, causal or not)

Pins (what each function is checked against, besides the product):
  compress/decompress: golden vectors produced by executing the reference's
    torch op sequence (tests/golden/make_golden.py) -- bit-exact.
  lloyd_max_closed_form: the scipy-quad fixture (centroids bit-equal, all
    boundaries but the middle one bit-equal), Max's 1960 table for 3 bits.
  layout: the reference's KAT (tests/test_vllm_integration.py:44-62).
  paged_decompress: closed form (sorted unique + per-row decompress).
  decode/prefill attention (tests/test_oracle_attention.py): torch's
    scaled_dot_product_attention in float64 over K/V dequantized by torch
    (GQA by repeat_interleave, explicit L - T + i causal mask); closed forms
    (zero context -> zeros, L = 1 -> V row, identical keys -> mean of V, two
    keys -> logistic weight of sm_scale * (s1 - s0)); prefill rows equal
    decode over the visible prefix; the q / out roundings against torch's
    own casts.  Mistakes planted through _kv_head, _visible and _scores
    (GQA map, mask offset, missing scale) and K/V left unrounded fail these
    checks.
  dense3_pack: a bit permutation (each of the 3 x 32 input bits of a group lands
    on its own output bit, checked bit by bit) and unpack inverts it, on all
    index values at every position (tests/test_oracle_golden.py).
  unfused_attention: K/V equal to torch's decompress-then-cast; a non-causal
    row equals the decode oracle over the whole context (two code paths);
    causal rows with fp32 K/V equal prefill_attention.
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "librq_oracle.so")
_lib = None

DTYPE_CODE = {"float16": 0, "bfloat16": 1, "float32": 2}


def build() -> str:
    """Compile rq_oracle.c (make) and return the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.rqo_compress.restype = ctypes.c_int64
        L.rqo_compress.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int,
                                   ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                   ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        L.rqo_decompress.restype = None
        L.rqo_decompress.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                     ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        L.rqo_row_norm.restype = ctypes.c_float
        L.rqo_row_norm.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.rqo_block_rotate.restype = None
        L.rqo_block_rotate.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p,
                                       ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------------------
# Raw-bits helpers (numpy has no bfloat16; arrays hold uint16 bit patterns)
# ---------------------------------------------------------------------------

def to_bits(t) -> tuple[np.ndarray, str]:
    """torch tensor (f16 / bf16 / f32, CPU) -> (contiguous numpy array of raw bits, dtype name)."""
    import torch
    name = str(t.dtype).replace("torch.", "")
    t = t.detach().contiguous().cpu()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16).copy(), name
    return t.float().numpy().copy(), "float32"


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to bf16 (nearest even) and return them as fp32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bfloat16":
        return bf16_round(x)
    if dtype == "float16":
        with np.errstate(over="ignore"):  # values beyond fp16 range become inf, as torch's cast does
            return x.astype(np.float32).astype(np.float16).astype(np.float32)
    return x.astype(np.float32)


# ---------------------------------------------------------------------------
# Compress / decompress (rq_oracle.c)
# ---------------------------------------------------------------------------

def compress(x_bits: np.ndarray, dtype: str, rot_t_even: np.ndarray, rot_t_odd: np.ndarray,
             boundaries: np.ndarray, blk: int, want_ties: bool = False):
    """(N, H, D) raw-bits input -> packed (N, H, D/2) u8, norms (N, H, 1) f32[, tie mask, tie count]."""
    N, H, D = x_bits.shape
    M = N * H
    x = np.ascontiguousarray(x_bits)
    re = np.ascontiguousarray(rot_t_even, dtype=np.float32)
    ro = np.ascontiguousarray(rot_t_odd, dtype=np.float32)
    b = np.ascontiguousarray(boundaries, dtype=np.float32)
    packed = np.zeros((M, D // 2), np.uint8)
    norms = np.zeros((M,), np.float32)
    ties = np.zeros((M, D), np.uint8) if want_ties else None
    n_ties = lib().rqo_compress(_ptr(x), DTYPE_CODE[dtype], M, D, _ptr(re), _ptr(ro), blk, _ptr(b), b.size,
                                _ptr(packed), _ptr(norms), _ptr(ties) if want_ties else None)
    out = (packed.reshape(N, H, D // 2), norms.reshape(N, H, 1))
    if want_ties:
        return out + (ties.reshape(N, H, D), int(n_ties))
    return out


def decompress_f32(packed: np.ndarray, norms: np.ndarray, centroids: np.ndarray) -> np.ndarray:
    """(N, H, D/2) u8 + (N, H, 1) f32 -> (N, H, D) fp32 products centroid * norm (before the cast)."""
    N, H, half = packed.shape
    D = 2 * half
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    n = np.ascontiguousarray(norms, dtype=np.float32).reshape(-1)
    c = np.ascontiguousarray(centroids, dtype=np.float32)
    out = np.zeros((N * H, D), np.float32)
    lib().rqo_decompress(_ptr(p), _ptr(n), N * H, D, _ptr(c), c.size, _ptr(out))
    return out.reshape(N, H, D)


def reference_cpu_compress(x, rot_T_even, rot_T_odd, boundaries):
    """The reference's CPU fallback compress as torch CPU ops, in its order
    (triton/isoquant_compress.py:161-190; planarquant_compress.py:157-186 is the
    same): norm, divide by norm + 1e-10, dense matmul with R^T, bucketize, clamp,
    nibble pack.  Used as the measured CPU baseline of compress (its bytes equal
    compress() above: the golden vectors pin both)."""
    import torch
    N, H, D = x.shape
    flat = x.reshape(N * H, D).float()
    raw_norms = torch.norm(flat, dim=-1, keepdim=True)
    normalized = flat / (raw_norms + 1e-10)
    rotation_T = torch.empty(D, D, dtype=torch.float32)
    rotation_T[:, 0::2] = rot_T_even
    rotation_T[:, 1::2] = rot_T_odd
    idx = torch.bucketize(normalized @ rotation_T, boundaries).clamp(0, 15).to(torch.uint8)
    packed = (idx[:, 0::2] << 4) | idx[:, 1::2]
    return packed.reshape(N, H, D // 2), raw_norms.reshape(N, H, 1)


def reference_cpu_decompress(packed, norms, centroids, dtype):
    """The reference's CPU fallback decompress as torch CPU ops
    (triton/isoquant_decompress.py:103-133): centroid lookup times norm, cast."""
    import torch
    N, H, half = packed.shape
    pf = packed.reshape(N * H, half)
    nf = norms.reshape(N * H, 1).float()
    out = torch.empty(N * H, 2 * half, dtype=torch.float32)
    out[:, 0::2] = centroids[(pf >> 4).long()] * nf
    out[:, 1::2] = centroids[(pf & 15).long()] * nf
    return out.reshape(N, H, 2 * half).to(dtype)


def decompress(packed, norms, centroids, dtype: str) -> np.ndarray:
    """Decompress and apply the reference's `.to(dtype)` cast; returns fp32 values of the rounded result."""
    return round_to(decompress_f32(packed, norms, centroids), dtype)


# ---------------------------------------------------------------------------
# Lloyd-Max codebook, closed form (lloyd_max.py:32-86 schedule)
# ---------------------------------------------------------------------------

def lloyd_max_closed_form(d: int, bits: int, max_iter: int = 200, tol: float = 1e-10):
    """Same iteration as the reference, with exact truncated-Gaussian means.

    Centroid update: E[X | a < X < b] = sigma^2 (phi(a) - phi(b)) / (Phi(b) - Phi(a))
    in units of sigma = 1/sqrt(d).  Returns float64 (centroids, boundaries, iterations).
    """
    n = 2 ** bits
    sigma = 1.0 / math.sqrt(d)
    lo, hi = -3.5 * sigma, 3.5 * sigma
    c = [lo + (hi - lo) * (i + 0.5) / n for i in range(n)]
    it = 0
    for it in range(max_iter):
        b = [(c[i] + c[i + 1]) / 2.0 for i in range(n - 1)]
        edges = [lo * 3] + b + [hi * 3]
        new = []
        for i in range(n):
            za, zb = edges[i] / sigma, edges[i + 1] / sigma
            den = 0.5 * (math.erfc(-zb / math.sqrt(2)) - math.erfc(-za / math.sqrt(2)))
            num = sigma * (math.exp(-0.5 * za * za) - math.exp(-0.5 * zb * zb)) / math.sqrt(2 * math.pi)
            new.append(num / den if den > 1e-15 else c[i])
        shift = max(abs(new[i] - c[i]) for i in range(n))
        c = new
        if shift < tol:
            break
    b = [(c[i] + c[i + 1]) / 2.0 for i in range(n - 1)]
    return np.array(c), np.array(b), it + 1


# ---------------------------------------------------------------------------
# Slot layout (rq_backend.py:155-188, :482-490)
# ---------------------------------------------------------------------------

def slot_layout(num_kv_heads: int, head_dim: int, dense3: bool = False) -> dict:
    """Byte offsets of the slot [K idx | K norms | V idx | V norms | pad]
    (rq_backend.py:155-188, :482-490); dense3: 3-bit indices in 3 D / 8 bytes
    per head (dense3_pack) instead of D / 2."""
    ib = 3 * head_dim // 8 if dense3 else head_dim // 2
    H = num_kv_heads
    k_idx_end = H * ib
    k_norm_end = k_idx_end + 4 * H
    v_idx_end = k_norm_end + H * ib
    v_norm_end = v_idx_end + 4 * H
    per_head = 1 << (2 * (ib + 4) - 1).bit_length()  # next_power_of_2(136) = 256 (dense: 104 -> 128)
    return dict(k_idx_end=k_idx_end, k_norm_end=k_norm_end, v_idx_end=v_idx_end,
                v_norm_end=v_norm_end, total_bytes=H * per_head, index_bytes=ib)


# ---------------------------------------------------------------------------
# Dense 3-bit index layout (opt-in, no counterpart in the reference)
# ---------------------------------------------------------------------------
# 32 indices i[0..31] of a head (dims 32G .. 32G+31) -> 12 bytes: dwords A, B, C,
# byte k (k = 0..3) of each:
#   A[k] = i[2k]      | i[2k+1] << 3  | (i[24+2k] & 3) << 6
#   B[k] = i[8+2k]    | i[9+2k] << 3  | (i[25+2k] & 3) << 6
#   C[k] = i[16+2k]   | i[17+2k] << 3 | (i[24+2k] >> 2) << 6 | (i[25+2k] >> 2) << 7

def nibbles_to_indices(packed: np.ndarray) -> np.ndarray:
    """(..., D/2) nibble-packed bytes -> (..., D) indices (byte j = idx[2j] << 4 | idx[2j+1])."""
    p = np.asarray(packed, np.uint8)
    return np.stack([p >> 4, p & 15], axis=-1).reshape(*p.shape[:-1], 2 * p.shape[-1])


def indices_to_nibbles(idx: np.ndarray) -> np.ndarray:
    i = np.asarray(idx, np.uint8)
    return ((i[..., 0::2] << 4) | i[..., 1::2]).astype(np.uint8)


def dense3_pack(packed: np.ndarray) -> np.ndarray:
    """(..., D/2) nibble-packed 3-bit indices -> (..., 3 D / 8) dense bytes."""
    i = nibbles_to_indices(packed).astype(np.uint8)
    if i.max(initial=0) > 7:
        raise ValueError("dense 3-bit layout needs indices < 8")
    g = i.reshape(*i.shape[:-1], -1, 32)
    k2 = 2 * np.arange(4)
    A = g[..., k2] | g[..., k2 + 1] << 3 | (g[..., 24 + k2] & 3) << 6
    B = g[..., 8 + k2] | g[..., 9 + k2] << 3 | (g[..., 25 + k2] & 3) << 6
    C = g[..., 16 + k2] | g[..., 17 + k2] << 3 | (g[..., 24 + k2] >> 2) << 6 | (g[..., 25 + k2] >> 2) << 7
    out = np.concatenate([A, B, C], axis=-1).astype(np.uint8)  # (..., groups, 12)
    return out.reshape(*i.shape[:-1], -1)


def dense3_unpack(dense: np.ndarray) -> np.ndarray:
    """(..., 3 D / 8) dense bytes -> (..., D/2) nibble-packed indices."""
    d = np.asarray(dense, np.uint8)
    g = d.reshape(*d.shape[:-1], -1, 12)
    A, B, C = g[..., 0:4], g[..., 4:8], g[..., 8:12]
    idx = np.zeros((*g.shape[:-1], 32), np.uint8)
    k2 = 2 * np.arange(4)
    idx[..., k2], idx[..., k2 + 1] = A & 7, (A >> 3) & 7
    idx[..., 8 + k2], idx[..., 9 + k2] = B & 7, (B >> 3) & 7
    idx[..., 16 + k2], idx[..., 17 + k2] = C & 7, (C >> 3) & 7
    idx[..., 24 + k2] = (A >> 6) | ((C >> 6) & 1) << 2
    idx[..., 25 + k2] = (B >> 6) | ((C >> 7) & 1) << 2
    return indices_to_nibbles(idx.reshape(*d.shape[:-1], -1))


def dense3_cache_to_nibbles(cache: np.ndarray, num_kv_heads: int, head_dim: int) -> np.ndarray:
    """A dense-3-bit cache -> the nibble-layout cache holding the same tokens (same
    indices and norms), so that the attention oracles read it unchanged."""
    NB, BS, _ = cache.shape
    kp, kn, vp, vn = read_slots(cache, num_kv_heads, head_dim, dense3=True)
    lay = slot_layout(num_kv_heads, head_dim)
    out = np.zeros((NB, BS, lay["total_bytes"]), np.uint8)
    compress_store(out, np.arange(NB * BS), kp, kn, vp, vn)
    return out


def compress_store(cache: np.ndarray, slot_mapping: np.ndarray, k_packed, k_norms, v_packed, v_norms,
                   dense3: bool = False) -> None:
    """Assemble rows [K idx | K norms | V idx | V norms | 0] and scatter (rq_backend.py:609-657).

    cache: (NB, BS, total_bytes) uint8, modified in place.  Slots < 0 are
    skipped (the reference would wrap them to the last slot).  k_packed /
    v_packed are nibble-packed; dense3 stores them in the dense 3-bit layout.
    """
    N, H, half = k_packed.shape
    lay = slot_layout(H, 2 * half, dense3)
    if dense3:
        k_packed, v_packed = dense3_pack(k_packed), dense3_pack(v_packed)
    rows = np.zeros((N, cache.shape[-1]), np.uint8)
    rows[:, :lay["k_idx_end"]] = k_packed.reshape(N, -1)
    rows[:, lay["k_idx_end"]:lay["k_norm_end"]] = np.ascontiguousarray(k_norms.reshape(N, H), np.float32).view(np.uint8)
    rows[:, lay["k_norm_end"]:lay["v_idx_end"]] = v_packed.reshape(N, -1)
    rows[:, lay["v_idx_end"]:lay["v_norm_end"]] = np.ascontiguousarray(v_norms.reshape(N, H), np.float32).view(np.uint8)
    flat = cache.reshape(-1, cache.shape[-1])
    for t in range(N):
        s = int(slot_mapping[t])
        if s >= 0:
            flat[s] = rows[t]


def read_slots(cache: np.ndarray, num_kv_heads: int, head_dim: int, dense3: bool = False):
    """Split a (NB, BS, total_bytes) cache into per-token K/V packed indices (nibble
    layout; a dense3 cache is unpacked) and norms."""
    NB, BS, TB = cache.shape
    H = num_kv_heads
    lay = slot_layout(H, head_dim, dense3)
    ib = lay["index_bytes"]
    flat = cache.reshape(NB * BS, TB)
    kp = flat[:, :lay["k_idx_end"]].reshape(-1, H, ib)
    kn = np.ascontiguousarray(flat[:, lay["k_idx_end"]:lay["k_norm_end"]]).view(np.float32).reshape(-1, H, 1)
    vp = flat[:, lay["k_norm_end"]:lay["v_idx_end"]].reshape(-1, H, ib)
    vn = np.ascontiguousarray(flat[:, lay["v_idx_end"]:lay["v_norm_end"]]).view(np.float32).reshape(-1, H, 1)
    if dense3:
        kp, vp = dense3_unpack(kp), dense3_unpack(vp)
    return kp, kn, vp, vn


def paged_decompress(cache, block_table, seq_lens, num_kv_heads, head_dim, k_cb, v_cb, dtype):
    """_decompress_cache_paged (rq_backend.py:763-852): unique referenced blocks, their
    decompressed K/V (U, BS, H, D) and the remapped block table."""
    NB, BS, _ = cache.shape
    bt = np.asarray(block_table)
    need = (np.asarray(seq_lens) + BS - 1) // BS
    mask = np.arange(bt.shape[1])[None, :] < need[:, None]
    uniq = np.unique(bt[mask])
    sel = cache[uniq]
    kp, kn, vp, vn = read_slots(sel, num_kv_heads, head_dim)
    k = decompress(kp, kn, k_cb, dtype).reshape(len(uniq), BS, num_kv_heads, head_dim)
    v = decompress(vp, vn, v_cb, dtype).reshape(len(uniq), BS, num_kv_heads, head_dim)
    remap = np.zeros(NB, np.int32)
    remap[uniq] = np.arange(len(uniq), dtype=np.int32)
    return k, v, remap[bt], len(uniq)


# ---------------------------------------------------------------------------
# Attention references (float64 over the exact dequantized K/V)
# ---------------------------------------------------------------------------

def _kv_rounding(kv_dtype, dtype):
    """The dtype K/V are rounded to: "q" (the default of the attention oracles) is the
    q dtype, as both reference kernels cast centroid * norm to it
    (fused_paged_rq_decode.py:146-147, :190-191; fused_paged_rq_int8_prefill.py:172,
    :224); None keeps the fp32 products (no rounding)."""
    return dtype if kv_dtype == "q" else kv_dtype


def gather_seq(cache, block_table_row, L, num_kv_heads, head_dim, k_cb, v_cb, kv_dtype=None):
    """K, V (L, H, D) fp64 dequantized (centroid * norm in fp32) for one sequence;
    with kv_dtype, rounded to that dtype as decompress() writes them (the pages
    _decompress_cache_paged hands to flash attention, rq_backend.py:737-852)."""
    NB, BS, TB = cache.shape
    nblk = (L + BS - 1) // BS
    pay = slot_layout(num_kv_heads, head_dim)["v_norm_end"]  # payload bytes (the padding is never read)
    phys = np.asarray(block_table_row)[:nblk]
    slots = cache[phys, :, :pay].reshape(nblk * BS, pay)[:L]  # whole blocks, then the first L slots
    kp, kn, vp, vn = read_slots(slots.reshape(L, 1, pay), num_kv_heads, head_dim)
    if kv_dtype is None:
        return decompress_f32(kp, kn, k_cb).astype(np.float64), decompress_f32(vp, vn, v_cb).astype(np.float64)
    return (decompress(kp, kn, k_cb, kv_dtype).astype(np.float64),
            decompress(vp, vn, v_cb, kv_dtype).astype(np.float64))


def block_width(R: np.ndarray) -> int:
    """Smallest width in (2, 4, 8, ..., D) for which R is block diagonal."""
    D = R.shape[0]
    idx = np.arange(D)
    blk = 2
    while blk < D:
        off = (idx[:, None] // blk) != (idx[None, :] // blk)
        if not np.any(R[off] != 0):
            return blk
        blk *= 2
    return D


def _block_rotate(x: np.ndarray, R: np.ndarray, transpose: bool) -> np.ndarray:
    """x @ R^T (transpose) or x @ R in fp32 with torch's CPU rounding order (rq_oracle.c)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    Rc = np.ascontiguousarray(R, dtype=np.float32)
    D = Rc.shape[0]
    rows = x.size // D
    out = np.zeros((rows, D), np.float32)
    sk, sj = (1, D) if transpose else (D, 1)
    lib().rqo_block_rotate(_ptr(x), rows, D, _ptr(Rc), sk, sj, block_width(Rc), _ptr(out))
    return out.reshape(x.shape)


def rotate_q(q_f32: np.ndarray, R: np.ndarray, dtype: str) -> np.ndarray:
    """q_rot = (q.float() @ R^T).to(dtype) (fused_paged_rq_decode.py:271), fp32 product in
    torch's CPU order."""
    return round_to(_block_rotate(q_f32, R, True), dtype)


def unrotate_out(out_rot: np.ndarray, R: np.ndarray, dtype: str) -> np.ndarray:
    """out = (out_rot.to(dtype).float() @ R).to(dtype) (fused_paged_rq_decode.py:201-206, :308)."""
    o = round_to(np.asarray(out_rot, np.float64).astype(np.float32), dtype)
    return round_to(_block_rotate(o, R, False), dtype)


def _kv_head(h: int, G: int, H: int) -> int:
    """KV head read by query head h (fused_paged_rq_decode.py:78: h // (H_Q / H_KV))."""
    return h // G


def _visible(pos_q: np.ndarray, L: int) -> np.ndarray:
    """(T, L) mask: key j is visible to a query at position p iff j <= p
    (fused_paged_rq_int8_prefill.py:187-189, with p = L - T + i)."""
    return np.arange(L)[None, :] <= np.asarray(pos_q)[:, None]


def _scores(qr: np.ndarray, K: np.ndarray, sm_scale: float) -> np.ndarray:
    """Scaled scores q . k * sm_scale (fused_paged_rq_decode.py:150-154 without the log2e
    change of base, which cancels in the softmax)."""
    return (qr @ K.T) * sm_scale


def decode_attention_rot(q, cache, block_table, seq_lens, num_kv_heads, head_dim, k_cb, v_cb, R, sm_scale, dtype,
                         kv_dtype="q"):
    """Rotated-space decode output in float64, before the output rounding:
    (B, HQ, D).  q: (B, HQ, D) fp32 values of the dtype-rounded query; K/V rounded
    to _kv_rounding(kv_dtype, dtype) (default: the q dtype, as the reference)."""
    kv_dtype = _kv_rounding(kv_dtype, dtype)
    B, HQ, D = q.shape
    G = HQ // num_kv_heads
    out = np.zeros((B, HQ, D))
    for b in range(B):
        L = int(seq_lens[b])
        if L == 0:
            continue  # empty context -> zeros (the reference: acc 0, l 1)
        qr = rotate_q(q[b], R, dtype).astype(np.float64)  # (HQ, D)
        K, V = gather_seq(cache, block_table[b], L, num_kv_heads, head_dim, k_cb, v_cb, kv_dtype)
        kv_of = np.array([_kv_head(h, G, num_kv_heads) for h in range(HQ)])
        for kvh in range(num_kv_heads):
            heads = np.nonzero(kv_of == kvh)[0]
            if heads.size == 0:
                continue
            S = _scores(qr[heads], np.ascontiguousarray(K[:, kvh, :]), sm_scale)  # (heads, L)
            P = np.exp(S - S.max(axis=1, keepdims=True))
            out[b, heads] = (P @ np.ascontiguousarray(V[:, kvh, :])) / P.sum(axis=1, keepdims=True)
    return out


def decode_attention(q, cache, block_table, seq_lens, num_kv_heads, head_dim, k_cb, v_cb, R, sm_scale, dtype,
                     kv_dtype="q"):
    """q: (B, HQ, D) fp32 values of the dtype-rounded query.  Returns (B, HQ, D) fp32 values."""
    o_rot = decode_attention_rot(q, cache, block_table, seq_lens, num_kv_heads, head_dim, k_cb, v_cb, R, sm_scale,
                                 dtype, kv_dtype)
    B, HQ, D = o_rot.shape
    return unrotate_out(o_rot.reshape(-1, D), R, dtype).reshape(B, HQ, D)


def prefill_attention_rot(q, cu_seqlens, cache, block_table, seq_lens, num_kv_heads, head_dim, k_cb, v_cb, R,
                          sm_scale, dtype, rows=None, causal=True, kv_dtype="q"):
    """Rotated-space prefill output in float64, before the output rounding: (T, HQ, D).

    Query i of sequence b sits at position seq_lens[b] - q_len_b + i; causal: it
    sees the keys at positions <= its own, else all seq_lens[b] keys.  rows
    (optional, sorted global query rows) restricts the work to those rows;
    the others stay zero.  K/V rounded to _kv_rounding(kv_dtype, dtype) (default:
    the q dtype, as the reference)."""
    kv_dtype = _kv_rounding(kv_dtype, dtype)
    T, HQ, D = q.shape
    G = HQ // num_kv_heads
    out = np.zeros((T, HQ, D))
    want = None if rows is None else np.asarray(rows)
    for b in range(len(seq_lens)):
        s0, s1 = int(cu_seqlens[b]), int(cu_seqlens[b + 1])
        L = int(seq_lens[b])
        T_b = s1 - s0
        if T_b == 0:
            continue
        local = np.arange(T_b) if want is None else want[(want >= s0) & (want < s1)] - s0
        if local.size == 0 or L == 0:
            continue
        K, V = gather_seq(cache, block_table[b], L, num_kv_heads, head_dim, k_cb, v_cb, kv_dtype)
        qr = rotate_q(q[s0 + local].reshape(-1, D), R, dtype).reshape(local.size, HQ, D).astype(np.float64)
        vis = _visible(L - T_b + local if causal else np.full(local.size, L - 1), L)
        Kc = [np.ascontiguousarray(K[:, j, :]) for j in range(num_kv_heads)]
        Vc = [np.ascontiguousarray(V[:, j, :]) for j in range(num_kv_heads)]
        for h in range(HQ):
            kvh = _kv_head(h, G, num_kv_heads)
            S = _scores(qr[:, h, :], Kc[kvh], sm_scale)  # (rows, L)
            S = np.where(vis, S, -np.inf)
            with np.errstate(invalid="ignore"):  # a row with no visible key (only a wrong mask) gives NaN
                S -= S.max(axis=1, keepdims=True)
                P = np.exp(S)
                out[s0 + local, h, :] = (P @ Vc[kvh]) / P.sum(axis=1, keepdims=True)
    return out


def prefill_attention(q, cu_seqlens, cache, block_table, seq_lens, num_kv_heads, head_dim, k_cb, v_cb, R,
                      sm_scale, dtype, rows=None, causal=True, kv_dtype="q"):
    """Attention of new tokens; query i of sequence b sits at position seq_lens[b] - q_len_b + i.
    Returns (T, HQ, D) fp32 values (rows outside `rows`, when given, are zero)."""
    o_rot = prefill_attention_rot(q, cu_seqlens, cache, block_table, seq_lens, num_kv_heads, head_dim, k_cb, v_cb,
                                  R, sm_scale, dtype, rows, causal, kv_dtype)
    T, HQ, D = o_rot.shape
    return unrotate_out(o_rot.reshape(-1, D), R, dtype).reshape(T, HQ, D)


def unfused_attention(q, cu_seqlens, cache, block_table, seq_lens, num_kv_heads, head_dim, k_cb, v_cb, R, sm_scale,
                      dtype, rows=None, causal=True):
    """The reference's non-fused path (rq_backend.py:937-1036): q_rot = q R^T rounded
    to the q dtype (:939-941, :981), K/V paged-decompressed to the q dtype
    (:737-852), flash_attn_varlen_func's attention with the bottom-right causal
    mask over seqused_k (:996-1030; here exact, in fp64), out_rot rounded to the
    q dtype, then out_rot R rounded (:1032-1034)."""
    return prefill_attention(q, cu_seqlens, cache, block_table, seq_lens, num_kv_heads, head_dim, k_cb, v_cb, R,
                             sm_scale, dtype, rows, causal, kv_dtype=dtype)
