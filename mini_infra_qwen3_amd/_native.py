"""ctypes binding of libmi_paged.so, the C ABI declared in include/mi_paged.h.

The library is loaded once, after torch, so that its HIP runtime dependency resolves to
the copy torch already mapped (one runtime per process: torch's streams are valid handles
for the library).  There is no fallback: if the library is missing or fails to load, every
data-plane call raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must be imported before the library; see module docstring)

LIBRARY_PATH = Path(__file__).resolve().with_name("libmi_paged.so")
ABI_VERSION = 4

MI_OK = 0
MI_ERR_INVALID_ARGUMENT = -1
MI_ERR_UNSUPPORTED = -2
MI_ERR_WORKSPACE = -3
MI_ERR_DEVICE = -4

_c_void_p_p = ctypes.POINTER(ctypes.c_void_p)
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p

# name -> (restype, argtypes); kept in the order of include/mi_paged.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "mi_abi_version": (_i32, []),
    "mi_last_error": (ctypes.c_char_p, []),
    "mi_reshape_and_cache": (
        _i32,
        [_c_void_p_p, _c_void_p_p, _i64, _i64, _i64, _i64, _i64, _i64, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64,
         _c_void_p_p, _c_void_p_p, _i32, _i64, _i32, _i32, _i32, _ptr],
    ),
    "mi_gather_blocks": (
        _i32,
        [_c_void_p_p, _c_void_p_p, _i64, _ptr, _i64, _i32, _i32, _c_void_p_p, _c_void_p_p, _i32, _i64, _ptr],
    ),
    "mi_paged_decode_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "mi_paged_decode_attention": (
        _i32,
        [_ptr, _i64, _ptr, _i64, _i64, _ptr, _ptr, _i64, _ptr, _i64, _i32, _ptr, _i64, _i32, _i32, _i32, _i32,
         _i32, ctypes.c_float, _ptr, _i64, _ptr],
    ),
    "mi_paged_decode_attention_fused": (
        _i32,
        [_ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr, _ptr, _ptr, _ptr, ctypes.c_float, _ptr, _i64, _ptr, _ptr,
         _i64, _ptr, _i64, _i32, _ptr, _i64, _i32, _i32, _i32, _i32, _i32, ctypes.c_float, _ptr, _ptr, _i64, _ptr],
    ),
    "mi_paged_decode_attention_noalloc": (
        _i32,
        [_ptr, _i64, _ptr, _i64, _i64, _ptr, _ptr, _i64, _ptr, _i64, _i32, _ptr, _i64, _i32, _i32, _i32, _i32,
         _i32, ctypes.c_float, _ptr],
    ),
    "mi_chunked_prefill_attention": (
        _i32,
        [_ptr, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _ptr, _i64,
         _ptr, _i64, _i32, _ptr, _ptr, _i64, _i32, _i32, _i32, _i32, _i32, _i32, ctypes.c_float, _ptr],
    ),
    "mi_paged_decode_attention_exact": (
        _i32,
        [_ptr, _i64, _ptr, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr, _ptr, _ptr, _ptr, ctypes.c_float, _ptr, _i64,
         _ptr, _ptr, _i64, _ptr, _i64, _i32, _ptr, _i64, _i32, _i32, _i32, _i32, _i32, ctypes.c_float, _ptr, _i64,
         _ptr],
    ),
    "mi_paged_decode_exact_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32]),
    "mi_chunked_prefill_attention_exact": (
        _i32,
        [_ptr, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _ptr, _i64,
         _ptr, _i64, _i32, _ptr, _ptr, _i64, _i32, _i32, _i32, _i32, _i32, _i32, ctypes.c_float, _ptr],
    ),
    "mi_mixed_paged_attention": (
        _i32,
        [_ptr, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _ptr, _i64, _i32, _i32, _i64, _ptr,
         _ptr, _i64, _i32, _ptr, _ptr, _i64, _i32, _ptr, _i64, _i32, _ptr, _i64, _ptr, _i64, _i32, _i32, _i32, _i32,
         ctypes.c_float, _ptr],
    ),
    "mi_mixed_paged_attention_exact": (
        _i32,
        [_ptr, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _ptr, _i64, _i32, _i32, _i64, _ptr,
         _ptr, _i64, _i32, _ptr, _ptr, _i64, _i32, _ptr, _i64, _i32, _ptr, _i64, _ptr, _i64, _i32, _i32, _i32, _i32,
         ctypes.c_float, _ptr],
    ),
    "mi_rms_norm": (_i32, [_ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i32, ctypes.c_float, _ptr]),
    "mi_qk_norm_rope": (
        _i32,
        [_ptr, _ptr, _ptr, _ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr, _ptr, _ptr, _ptr, _i64, _i32, _i32, _i32,
         ctypes.c_float, _ptr, _i64, _ptr, _ptr, _i64, _ptr],
    ),
    "mi_silu_mul": (_i32, [_ptr, _i64, _ptr, _i64, _ptr, _i64, _i64, _i32, _ptr]),
    "mi_argmax_rows": (_i32, [_ptr, _ptr, _i64, _i32, _i64, _ptr]),
    "mi_pack_blocks": (_i32, [_ptr, _c_void_p_p, _c_void_p_p, _i64, _ptr, _i64, _i32, _i64, _ptr]),
    "mi_unpack_blocks": (_i32, [_c_void_p_p, _c_void_p_p, _i64, _ptr, _ptr, _i64, _i32, _i64, _ptr]),
}


class NativeLibraryError(RuntimeError):
    """libmi_paged.so is missing, stale or could not be loaded."""


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def _hip_runtimes_mapped() -> set[str]:
    try:
        with open("/proc/self/maps") as maps:
            return {line.split()[-1] for line in maps if "libamdhip64" in line}
    except OSError:
        return set()


def load() -> ctypes.CDLL:
    """Loads (once) and returns the library with argument types declared."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIBRARY_PATH.exists():
            raise NativeLibraryError(
                f"{LIBRARY_PATH} not found: build it with `python -m mini_infra_qwen3_amd.build` "
                "(the paged-KV data plane has no CPU or torch fallback)"
            )
        try:
            lib = ctypes.CDLL(str(LIBRARY_PATH))
        except OSError as exc:
            raise NativeLibraryError(f"cannot load {LIBRARY_PATH}: {exc}") from exc
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.mi_abi_version()
        if version != ABI_VERSION:
            raise NativeLibraryError(f"{LIBRARY_PATH} has ABI {version}, expected {ABI_VERSION}: rebuild it")
        runtimes = _hip_runtimes_mapped()
        if len(runtimes) > 1:
            raise NativeLibraryError(f"two HIP runtimes mapped in this process: {sorted(runtimes)}")
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    """Raises the Python error matching a negative ABI status (ValueError for bad arguments)."""
    if rc == MI_OK:
        return
    message = load().mi_last_error().decode(errors="replace") or what
    if rc in (MI_ERR_INVALID_ARGUMENT, MI_ERR_UNSUPPORTED, MI_ERR_WORKSPACE):
        raise ValueError(message)
    raise RuntimeError(message)


def pointer_array(ptrs: list[int]) -> ctypes.Array:
    return (ctypes.c_void_p * len(ptrs))(*ptrs)
