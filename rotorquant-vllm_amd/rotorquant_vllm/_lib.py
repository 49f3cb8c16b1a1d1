"""Loader for librq_hip.so, the gfx950 HIP library behind the C ABI in include/rq_abi.h.

torch is imported first so that its HIP runtime (libamdhip64.so.7) is the one
the library binds to; the library then launches on torch's current stream.
There is no fallback: if the library is missing or fails to load, every op
raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime the library links against)

LIB_NAME = "librq_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

DTYPE_F16, DTYPE_BF16, DTYPE_F32 = 0, 1, 2
_DTYPE_CODE = {torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16, torch.float32: DTYPE_F32}

_c_i32, _c_i64, _c_f32, _c_p = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p

_SIGNATURES = {
    "rq_abi_version": (_c_i32, []),
    "rq_last_error": (ctypes.c_char_p, []),
    "rq_compress": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i32, _c_p, _c_p, _c_i32, _c_p, _c_i32, _c_p, _c_p, _c_p]),
    "rq_compress_store": (_c_i32, [_c_p, _c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32,
                                   _c_p, _c_p, _c_i64, _c_i32, _c_i64, _c_i64, _c_i32, _c_p, _c_p, _c_i32, _c_p,
                                   _c_i32, _c_p, _c_i32, _c_p]),
    "rq_decompress": (_c_i32, [_c_p, _c_p, _c_i64, _c_i32, _c_p, _c_i32, _c_p, _c_i32, _c_p]),
    "rq_paged_decompress_workspace_bytes": (_c_i64, [_c_i64]),
    "rq_paged_decompress": (_c_i32, [_c_p, _c_i64, _c_i32, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_i64,
                                     _c_i64, _c_i64, _c_p, _c_p, _c_i32, _c_p, _c_i32, _c_p, _c_p, _c_i32, _c_i64,
                                     _c_p, _c_p, _c_p, _c_i64, _c_p]),
    "rq_fused_decode_workspace_bytes": (_c_i64, [_c_i64, _c_i32, _c_i32, _c_i64]),
    "rq_fused_decode": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i32, _c_i64, _c_i64, _c_p, _c_i64, _c_i32, _c_i64, _c_i64,
                                 _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_i32, _c_p,
                                 _c_i32, _c_p, _c_i32, _c_f32, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_p]),
    "rq_fused_decode_timed": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i32, _c_i64, _c_i64, _c_p, _c_i64, _c_i32, _c_i64,
                                       _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_p,
                                       _c_i32, _c_p, _c_i32, _c_p, _c_i32, _c_f32, _c_p, _c_i64, _c_i64, _c_p,
                                       _c_i64, _c_p, _c_p, _c_p]),
    "rq_fused_decode_noalloc": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i32, _c_i64, _c_i64, _c_p, _c_i64, _c_i32, _c_i64,
                                         _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_p,
                                         _c_i32, _c_p, _c_i32, _c_p, _c_i32, _c_f32, _c_p, _c_i64, _c_i64, _c_p]),
    "rq_int8_prefill_workspace_bytes": (_c_i64, [_c_i64, _c_i32, _c_i64]),
    "rq_int8_prefill": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i32, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_i64,
                                 _c_i32, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_i64, _c_p, _c_i64,
                                 _c_p, _c_i32, _c_p, _c_i32, _c_p, _c_i32, _c_f32, _c_p, _c_i64, _c_i64, _c_p, _c_i64,
                                 _c_p]),
    "rq_paged_attention": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i32, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i32, _c_p,
                                    _c_i64, _c_i32, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_i64,
                                    _c_p, _c_p, _c_i32, _c_p, _c_i32, _c_p, _c_i32, _c_f32, _c_p, _c_i64, _c_i64, _c_p]),
    "rq_paged_prefill_workspace_bytes": (_c_i64, [_c_i64, _c_i32, _c_i64]),
    "rq_paged_prefill": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i32, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i32, _c_p,
                                  _c_i64, _c_i32, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_i64,
                                  _c_p, _c_i64, _c_p, _c_i32, _c_p, _c_i32, _c_p, _c_i32, _c_f32, _c_p, _c_i64, _c_i64,
                                  _c_p, _c_i64, _c_p]),
}

EXPORTED = tuple(_SIGNATURES)

_lib = None
_load_error: str | None = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library (once) and attach the C signatures.  Raises on failure."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        _load_error = f"{path} not found: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
        raise ImportError(_load_error)
    try:
        lib = ctypes.CDLL(path)
    except OSError as exc:
        _load_error = f"{path} failed to load: {exc}"
        raise ImportError(_load_error) from exc
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except ImportError:
        return False


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}") from None


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().rq_last_error().decode(errors="replace")
        if rc == 1:
            raise ValueError(f"{what}: {msg}")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
