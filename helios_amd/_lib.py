"""ctypes binding of libheliosattn.so (declared in include/helios_attn.h).

torch is imported first on purpose: torch ships its own copy of the HIP
runtime (soname libamdhip64.so.7), and the dynamic linker only reuses it for
this library if it is already loaded, so that both see the same streams.
There is no fallback: if the library or a GPU is missing, every entry point
raises RuntimeError (like helios' Triton wrapper, triton_attn.py:146-150).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "libheliosattn.so"

HPA_OK = 0
HPA_ERR_ARG = 1
HPA_ERR_UNSUPPORTED = 2
HPA_ERR_WORKSPACE = 3
HPA_ERR_LAUNCH = 4

# bytes of the static per-GPU scratch of hpa_paged_decode_noalloc
HPA_NOALLOC_SCRATCH_BYTES = 64 << 20

HPA_F32 = 0
HPA_F16 = 1
HPA_BF16 = 2
HPA_I8 = 3

DTYPE_CODE = {
    torch.float32: HPA_F32,
    torch.float16: HPA_F16,
    torch.bfloat16: HPA_BF16,
    torch.int8: HPA_I8,
}

_c_int = ctypes.c_int
_c_size = ctypes.c_size_t
_c_ptr = ctypes.c_void_p
_c_float = ctypes.c_float

# name -> (restype, argtypes); mirrors include/helios_attn.h
SIGNATURES = {
    "hpa_version": (_c_int, []),
    "hpa_last_error": (ctypes.c_char_p, []),
    "hpa_decode_workspace_size": (_c_size, [_c_int] * 7),
    "hpa_paged_decode": (
        _c_int,
        [_c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int,
         _c_ptr, _c_int, _c_ptr, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_int, _c_float, _c_int, _c_ptr, _c_size, _c_ptr],
    ),
    "hpa_paged_decode_noalloc": (
        _c_int,
        [_c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int,
         _c_ptr, _c_int, _c_ptr, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_int, _c_float, _c_int, _c_ptr],
    ),
    "hpa_paged_prefill": (
        _c_int,
        [_c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int,
         _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_int, _c_int, _c_int, _c_float, _c_ptr],
    ),
    "hpa_kv_write": (
        _c_int,
        [_c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int,
         _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_ptr],
    ),
    "hpa_kv_write_rope": (
        _c_int,
        [_c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int,
         _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_ptr, _c_ptr, _c_int, _c_ptr],
    ),
    "hpa_kv_gather": (
        _c_int,
        [_c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_int, _c_ptr,
         _c_ptr, _c_int, _c_int, _c_int, _c_int, _c_int, _c_ptr],
    ),
    "hpa_copy_blocks": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_int, _c_int, _c_size,
         _c_size, _c_ptr],
    ),
    "hpa_step_tables": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_int, _c_ptr, _c_int, _c_int, _c_ptr, _c_int, _c_ptr],
    ),
}

_lib: Optional[ctypes.CDLL] = None


def load_library(path: Optional[os.PathLike] = None) -> ctypes.CDLL:
    """Load (once) and type the shared library. Raises RuntimeError if absent."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"{p} is not built; run `python -m helios_amd.build` (hipcc, gfx950)"
        )
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def hip_available() -> bool:
    """True when the library is built and a GPU is visible."""
    return LIB_PATH.exists() and torch.cuda.is_available()


def lib() -> ctypes.CDLL:
    if not torch.cuda.is_available():
        raise RuntimeError(
            "helios_amd paged attention runs on an MI355X (gfx950) GPU; no GPU is visible"
        )
    return load_library()


def check(status: int, what: str) -> None:
    """Map a C-ABI status to an exception (helios' runner turns both into
    ExecFault(CUDA_ERROR), reference exec/runner.py:139-147)."""
    if status == HPA_OK:
        return
    msg = load_library().hpa_last_error().decode(errors="replace")
    raise RuntimeError(f"{what} failed (status {status}): {msg}")


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()
