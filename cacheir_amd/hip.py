"""ctypes binding of ``libcacheir_hip.so`` (declared in ``include/cacheir_hip.h``).

The library is loaded after ``torch`` so it binds to the HIP runtime torch already
loaded.  There is no CPU fallback: if the library is missing or a call fails, a
``RuntimeError`` names the entry point and the library's error text.

Tensor arguments are torch tensors on the GPU; their ``data_ptr()`` is passed.
The stream defaults to torch's current stream (a ``hipStream_t`` on ROCm builds).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

# CACHEIR_HIP_LIB selects another build of the same library (e.g. one compiled with other options).
LIB_PATH = Path(os.environ.get("CACHEIR_HIP_LIB") or Path(__file__).resolve().parent / "_lib" / "libcacheir_hip.so")

CIR_F32 = 0
CIR_F16 = 1
CIR_Q4_0 = 2
CIR_Q8_0 = 8
CIR_I4_ROW = 64  # the reference's per-row asymmetric int4 packing
CIR_I8_ROW = 65  # ... and int8
ATTENTION_NOALLOC_MAX_BYTES = 16 << 20  # CIR_ATTENTION_NOALLOC_MAX_BYTES
GEMM_PARTIALS, GEMM_SWIGLU, GEMM_ARGMAX, GEMM_ATTN_MERGE = 0, 1, 2, 3  # cir_qgemm_plan ops

_c_int, _c_size, _c_float, _vp = ctypes.c_int, ctypes.c_size_t, ctypes.c_float, ctypes.c_void_p

# name -> (restype, argtypes)
_SIGNATURES = {
    "cir_version": (ctypes.c_char_p, []),
    "cir_last_error_string": (ctypes.c_char_p, []),
    "cir_paged_attention_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "cir_paged_decode_attention": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_size, _c_int, _c_int, _c_int, _c_int,
                                            _c_int, _c_int, _c_float, _c_int, _vp]),
    "cir_paged_decode_attention_noalloc": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int,
                                                    _c_int, _c_int, _c_float, _c_int, _vp]),
    "cir_paged_decode_attention_qkv": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_size, _c_int,
                                                _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _vp]),
    "cir_paged_decode_splits": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "cir_paged_decode_attention_qkv_parts": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_size, _c_int,
                                                      _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _vp]),
    "cir_paged_prefill_attention": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_size, _c_int, _c_int, _c_int, _c_int,
                                             _c_int, _c_int, _c_int, _c_float, _c_int, _vp]),
    "cir_qweight_tiled_bytes": (_c_size, [_c_int, _c_int, _c_int]),
    "cir_qweight_repack": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _vp]),
    "cir_qweight_repack_rows": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp]),
    "cir_dequant": (_c_int, [_vp, _c_int, _c_int, _vp, _c_int, _c_int, _vp]),
    "cir_qgemm_splits": (_c_int, [_c_int, _c_int, _c_int]),
    "cir_qgemm_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int]),
    "cir_qgemm": (_c_int, [_vp, _c_int, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp]),
    "cir_qgemm_plan": (ctypes.c_char_p, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "cir_qgemm_attn": (_c_int, [_vp, _vp, _c_int, _c_int, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp]),
    "cir_qgemm_swiglu": (_c_int, [_vp, _c_int, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp]),
    "cir_qgemm_argmax_workspace_bytes": (_c_size, [_c_int, _c_int]),
    "cir_qgemm_argmax": (_c_int, [_vp, _c_int, _vp, _c_int, _vp, _vp, _c_size, _c_int, _c_int, _c_int, _vp]),
    "cir_gemm_f32": (_c_int, [_vp, _c_int, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp]),
    "cir_epilogue_store": (_c_int, [_vp, _c_int, _vp, _vp, _c_int, _c_int, _c_int, _vp]),
    "cir_epilogue_residual_rmsnorm": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _c_int, _c_float, _vp, _c_int, _c_int,
                                               _c_int, _vp]),
    "cir_epilogue_swiglu": (_c_int, [_vp, _c_int, _vp, _c_int, _c_int, _c_int, _vp]),
    "cir_stream_read": (_c_int, [_vp, _c_size, _c_int, _c_int, _c_int, _vp, _c_size, _c_int, _vp, _vp]),
    "cir_epilogue_qkv_rope_append": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _c_int, _vp, _c_int, _vp, _vp, _c_int, _c_int,
                                              _c_int, _c_int, _c_int, _c_int, _c_int, _vp]),
    "cir_embedding": (_c_int, [_vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp]),
    "cir_rmsnorm": (_c_int, [_vp, _c_int, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_float, _vp]),
    "cir_add": (_c_int, [_vp, _vp, _vp, _c_int, _c_size, _vp]),
    "cir_cast": (_c_int, [_vp, _c_int, _vp, _c_int, _c_size, _vp]),
    "cir_argmax": (_c_int, [_vp, _c_int, _vp, _c_int, _c_int, _vp]),
}

_lib: ctypes.CDLL | None = None


def library_path() -> Path:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises RuntimeError if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"cacheir_amd HIP library not found at {LIB_PATH}; build it with `python -m cacheir_amd.build` "
            "(there is no CPU fallback)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return CIR_F32
    if dt == torch.float16:
        return CIR_F16
    raise TypeError(f"unsupported dtype {dt} (float32 or float16)")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(stream: torch.cuda.Stream | None = None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def call(name: str, *args) -> None:
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        msg = (lib.cir_last_error_string() or b"").decode()
        raise RuntimeError(f"{name} failed with status {status}: {msg}")


def size_call(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))
