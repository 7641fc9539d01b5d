"""ctypes binding of ``libfast_mimi_amd.so`` (the C ABI in ``include/fast_mimi_amd.h``).

The library is loaded lazily on first use and never replaced by a Python or
PyTorch fallback: if it is missing or fails to load, every GPU entry point
raises ``NativeLibraryError``.  Each wrapper passes raw device pointers, sizes
and the caller's HIP stream, and maps a non-zero status to ``NativeError``.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIBRARY_PATH = Path(
    os.environ.get("FAST_MIMI_AMD_LIBRARY", Path(__file__).resolve().parent / "libfast_mimi_amd.so")
)
ABI_VERSION = 1

# Flags shared with csrc/fm_common.h.
ELU_IN = 1
REPLICATE = 2
EPI_ELU = 4
EPI_GELU = 8
EPI_RES_ADD = 16
EPI_RES_SCALE = 32
WEIGHTS_X6 = 64
ACT_EXP = 128  # residual blocks: ELU as e^x - 1 (decoder-side calls)

_STATUS = {1000: "bad argument", 1001: "workspace too small", 1002: "unsupported shape",
           1003: "input larger than the fixed scratch of an allocation-free entry point"}


class NativeLibraryError(RuntimeError):
    """The HIP library could not be loaded (not built, or no ROCm runtime)."""


class NativeError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_long
_F = ctypes.c_float
_S = ctypes.c_size_t

_SIGNATURES = {
    "fm_abi_version": ([], _I),
    "fm_gemm_last_plan": ([ctypes.c_char_p, _I], _I),
    "fm_split_weights": ([_P, _I, _I, _P, _P], _I),
    "fm_conv1d": ([_P, _I, _I, _I, _P, _P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _S, _P], _I),
    "fm_conv1d_rows_supported": ([_I, _I, _I, _I], _I),
    "fm_conv1d_rows": ([_P, _I, _I, _I, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P], _I),
    "fm_conv1d_valid": ([_P, _I, _I, _I, _P, _P, _I, _I, _I, _I, _P, _P, _P, _S, _P], _I),
    "fm_conv_transpose1d": ([_P, _I, _I, _I, _P, _P, _I, _I, _I, _I, _P, _P, _P, _S, _P], _I),
    "fm_linear": ([_P, _I, _I, _P, _I, _I, _P, _P, _P, _P, _S, _P], _I),
    "fm_linear_rope": ([_P, _I, _I, _P, _I, _I, _P, _P, _I, _I, _P, _P, _S, _P], _I),
    "fm_row_linear_supported": ([_I, _I], _I),
    "fm_row_linear": ([_P, _I, _I, _P, _P, _F, _P, _I, _I, _P, _P, _P, _P, _I, _I, _P, _P], _I),
    "fm_row_linear_packed": ([_P, _I, _I, _P, _P, _F, _P, _I, _I, _P, _P, _P, _P, _I, _I, _P, _P], _I),
    "fm_pack_row_weights": ([_P, _I, _I, _P, _P], _I),
    "fm_row_linear_packed_upsample": ([_P, _I, _I, _P, _I, _I, _P, _P, _P], _I),
    "fm_apply_rope": ([_P, _L, _I, _I, _I, _P, _P, _I, _P], _I),
    "fm_layer_norm": ([_P, _P, _P, _L, _I, _F, _P, _P], _I),
    "fm_window_attention": ([_P, _I, _I, _I, _I, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P, _I, _P], _I),
    "fm_window_attention_rows": ([_P, _I, _I, _I, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P, _I, _P], _I),
    "fm_rvq_prepare_codebook": ([_P, _P, _I, _I, _F, _P, _P, _P, _P], _I),
    "fm_rvq_workspace_bytes": ([_I, _I, _I], _S),
    "fm_rvq_encode": ([_P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _P, _S, _P], _I),
    "fm_rvq_split_workspace_bytes": ([_I, _I, _I], _S),
    "fm_rvq_encode_split": ([_P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _P, _S, _P], _I),
    "fm_rvq_noalloc_scratch_bytes": ([], _S),
    "fm_rvq_encode_split_noalloc": ([_P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _P], _I),
    "fm_rvq_decode": ([_P, _I, _I, _I, _I, _P, _I, _I, _P, _P], _I),
    "fm_upsample_depthwise": ([_P, _I, _I, _I, _P, _I, _I, _P, _P], _I),
    "fm_copy_buffers": ([_P, _P, _S, _P, _P, _S, _P], _I),
    "fm_resblock_supported": ([_I], _I),
    "fm_resblock": ([_P, _I, _I, _I, _P, _P, _P, _P, _I, _P, _P], _I),
    "fm_conv_resblock64": ([_P, _I, _I, _P, _P, _P, _P, _P, _P, _I, _P, _P], _I),
    "fm_resblock64_conv_workspace_bytes": ([_I, _I], _S),
    "fm_resblock64_conv": ([_P, _I, _I, _P, _P, _P, _P, _I, _P, _P, _I, _P, _P, _S, _P], _I),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def library() -> ctypes.CDLL:
    """Load (once) and return the HIP library, or raise ``NativeLibraryError``."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIBRARY_PATH.is_file():
            raise NativeLibraryError(
                f"{LIBRARY_PATH} is missing; build it with `python fast-mimi_amd/build_native.py`"
            )
        try:
            lib = ctypes.CDLL(str(LIBRARY_PATH))
        except OSError as exc:  # pragma: no cover - depends on the ROCm runtime
            raise NativeLibraryError(f"cannot load {LIBRARY_PATH}: {exc}") from exc
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        version = lib.fm_abi_version()
        if version != ABI_VERSION:
            raise NativeLibraryError(f"ABI version {version} != expected {ABI_VERSION}; rebuild")
        _lib = lib
        return lib


def check(status: int, name: str) -> None:
    if status != 0:
        raise NativeError(f"{name} failed: {_STATUS.get(status, f'hipError_t {status}')}")


def call(name: str, *args) -> None:
    check(getattr(library(), name)(*args), name)


def last_gemm_plan() -> str:
    """Kernel, tiles and K splits of the last GEMM-engine call on this thread."""
    buf = ctypes.create_string_buffer(160)
    check(library().fm_gemm_last_plan(buf, len(buf)), "fm_gemm_last_plan")
    return buf.value.decode()
