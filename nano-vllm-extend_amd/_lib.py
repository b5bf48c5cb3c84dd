"""ctypes binding of libgdn_mi355x.so (the C ABI declared in include/gdn_mi355x.h).

The library links against the HIP runtime bundled with torch, so torch is
imported first: its libamdhip64.so.7 is then already resident and satisfies
the library's dependency.  Missing library -> GDNLibraryError, never a
silent fallback.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

LIB_PATH = Path(os.environ.get("GDN_MI355X_LIB", Path(__file__).resolve().parent / "lib" / "libgdn_mi355x.so"))
ABI_VERSION = 4

GDN_OK = 0
GDN_ERR_INVALID_ARG = -1
GDN_ERR_UNSUPPORTED = -2
GDN_ERR_SCRATCH = -3
NOALLOC_SCRATCH_BYTES = 128 << 20   # GDN_NOALLOC_SCRATCH_BYTES


class GDNLibraryError(RuntimeError):
    """The HIP extension is missing or failed to load."""


class GDNKernelError(RuntimeError):
    """An entry point rejected its arguments or its launch failed."""


_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> argtypes (order and meaning as in include/gdn_mi355x.h)
SIGNATURES: dict[str, list] = {
    "gdn_abi_version": [],
    "gdn_g_beta": [_p, _p, _p, _p, _i32, _p, _p, _p, _i64, _i32, _p],
    "gdn_conv_varlen": [_p, _i64, _p, _i64, _i64, _p, _p, _p, _i32, _p, _p, _i32, _i64, _i32, _i32, _p],
    "gdn_conv_decode": [_p, _i64, _p, _i64, _i64, _p, _p, _p, _i64, _i32, _i32, _i32, _p],
    "gdn_conv_padded": [_p, _i64, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _i32, _i32, _i32, _i32, _p],
    "gdn_chunk_prefill": [_p, _i64, _p, _i64, _p, _i64, _p, _p, _p, _p, _p, _i64, _p, _p, _i32, _i32, _i64,
                          _i32, _i32, _i32, _f32, _i32, _p, _p, _i64, _p],
    "gdn_chunk_prefill_workspace_size": [_i64, _i32, _i32, _i32],
    "gdn_set_column_split": [_i32],
    "gdn_conv_chunk_prefill": [_p, _i64, _p, _i64, _i64, _p, _p, _p, _p, _p, _i32, _p, _p, _p, _p, _i64, _p, _p,
                               _i32, _i32, _p, _i32, _i64, _i32, _i32, _i32, _f32, _i32, _p, _p, _i64, _p],
    "gdn_conv_chunk_prefill_workspace_size": [_i64, _i32, _i32, _i32],
    "gdn_conv_chunk_prefill_noalloc": [_p, _i64, _p, _i64, _i64, _p, _p, _p, _p, _p, _i32, _p, _p, _p, _p, _i64,
                                       _p, _p, _i32, _i32, _i64, _i32, _i32, _i32, _f32, _i32, _p, _p],
    "gdn_recurrent": [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _i64, _p, _i64,
                      _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _p, _p, _i32, _p],
    "gdn_recurrent_decode_fused": [_p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _p, _p, _p, _p, _p, _i32,
                                   _p, _i64, _p, _p, _i32, _i32, _i32, _i32, _f32, _i32, _p, _i64, _p, _f32,
                                   _p],
    "gdn_state_commit": [_p, _i64, _p, _p, _p, _i32, _i32, _i32, _i32, _p],
    "gdn_gemm_bf16": [_p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32, _p, _p, _p, _p, _i32, _i32, _i32, _p],
    "gdn_gemm_bf16_cols": [_p, _i64, _p, _i64, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p, _p, _i32, _i32,
                           _i32, _p],
    "gdn_rmsnorm_gated": [_p, _i64, _p, _i64, _p, _p, _i64, _i32, _i32, _f32, _p],
    "gdn_state_tile_pass": [_p, _i64, _p, _i32, _i32, _i32, _p],
    "gdn_state_tile_copy": [_p, _p, _i64, _p, _i32, _i32, _i32, _p],
    "gdn_rmsnorm_gated_ranges": [_p, _i64, _p, _i64, _p, _p, _i64, _p, _i32, _i64, _i32, _i32, _f32, _p],
}

# entry points whose return type is not int (status)
RESTYPES = {"gdn_chunk_prefill_workspace_size": ctypes.c_int64,
            "gdn_conv_chunk_prefill_workspace_size": ctypes.c_int64}

_LIB: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the library once and bind every entry point's argtypes."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise GDNLibraryError(
            f"{LIB_PATH} not found: build it with `python nano-vllm-extend_amd/build.py` "
            "(or __graft_entry__.build()); there is no fallback path")
    try:
        lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
    except OSError as e:  # pragma: no cover - environment dependent
        raise GDNLibraryError(f"cannot load {LIB_PATH}: {e}") from e
    # the version first: a library of another version may lack entry points
    lib.gdn_abi_version.argtypes = []
    lib.gdn_abi_version.restype = ctypes.c_int
    v = lib.gdn_abi_version()
    if v != ABI_VERSION:
        raise GDNLibraryError(f"ABI mismatch: library {v}, bindings {ABI_VERSION}")
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = RESTYPES.get(name, ctypes.c_int)
    _LIB = lib
    return lib


def check(name: str, status: int) -> None:
    if status == GDN_OK:
        return
    if status == GDN_ERR_INVALID_ARG:
        raise GDNKernelError(f"{name}: invalid argument (shape / stride / alignment rejected)")
    if status == GDN_ERR_UNSUPPORTED:
        raise GDNKernelError(f"{name}: unsupported configuration (head dim must be 64 or 128, conv width 4)")
    if status == GDN_ERR_SCRATCH:
        raise GDNKernelError(f"{name}: the call needs more scratch than the allocation-free entry point's fixed "
                             f"{NOALLOC_SCRATCH_BYTES >> 20} MiB array holds; use the workspace entry point")
    raise GDNKernelError(f"{name}: HIP launch failed with hipError_t {status}")


def call(name: str, *args) -> None:
    """Invoke an entry point and raise on a non-zero status."""
    lib = load()
    check(name, getattr(lib, name)(*args))


def ptr(t) -> int | None:
    """Device pointer of a tensor (None -> NULL)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_handle(device) -> int:
    """hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream
