"""ctypes binding of the gfx950 C ABI (include/cubic_mi355x.h).

The library is built in-tree by ``cubic_serve_amd.build`` into
``cubic_serve_amd/_lib/libcubic_mi355x.so``.  There is no CPU or Python
fallback: every operator raises if the library is missing.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

_LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libcubic_mi355x.so"
_lib: ctypes.CDLL | None = None

P = ctypes.c_void_p
I32 = ctypes.c_int
I64 = ctypes.c_int64

ABI_VERSION = 6  # cubic_abi_version() of the library these signatures describe

# name -> (restype, argtypes); mirrors include/cubic_mi355x.h
SIGNATURES: dict[str, tuple] = {
    "cubic_abi_version": (I32, []),
    "cubic_last_error": (ctypes.c_char_p, []),
    "cubic_prepared_words": (I32, [I64, I64, I32, I32, P, P]),
    "cubic_prepare_scratch_bytes": (I64, [I64, I64, I32]),
    "cubic_prepare_weight": (I32, [I32, P, P, P, P, P, P, P, P, I64, I64, I32, I32, I32, I32, P, I64,
                                   P, P, P]),
    "cubic_gemm_workspace_bytes": (I64, [I64, I64, I64, I32]),
    "cubic_gemm_group_workspace_bytes": (I64, [I64, I32, I64, I64, I32]),
    "cubic_gemm_grouped_workspace_bytes": (I64, [I64, I64, I64, I64, I32]),
    "cubic_gemm_group": (I32, [P, I64, P, P, I64, I32, I64, I64, I32, I32, I32, P, P, P, I64, P]),
    "cubic_gemm": (I32, [P, I64, P, P, I64, I64, I64, I32, I32, I32, P, I64, P, I64, P]),
    "cubic_gemm_grouped": (I32, [P, I64, P, P, I64, I64, I64, I64, I32, I32, I32, P, I64, P, I64, P,
                                 I64, P]),
    "cubic_moe_pad_routes": (I32, [P, P, P, P, P, I32, I32, I32, P, P, P, P]),
    "cubic_moe_max_blocks": (I64, [I64, I32, I32]),
    "cubic_moe_gemm": (I32, [P, I64, P, P, I64, I64, P, P, P, I64, I32, I32, I32, I64, I64, I32, I32, I32,
                             P, I64, P]),
    "cubic_embedding": (I32, [P, I32, I64, I32, P, P, P, P, P, P, P, P, I64, I64, I32, I32, I32, P,
                              I32, P]),
    "cubic_moe_route": (I32, [P, I32, P, P, I32, I32, I32, P, P, P, P, I32, P]),
    "cubic_moe_compact": (I32, [P, I32, I32, I32, I32, P, P, P, P, P, P]),
    "cubic_candidates_workspace_bytes": (I64, [I32, I32]),
    "cubic_candidates": (I32, [P, I32, I64, I32, I32, I64, P, I32, P, P, I32, I32, I32, P, P, P, I64, P]),
    "cubic_verify_candidates": (I32, [P, P, P, P, P, P, P, P, P, P, P, P, P, I32, I32, I32, I32,
                                      I32, I32, P, P]),
    "cubic_root_sample": (I32, [P, I32, P, P, P, P, P, P, P, I32, I32, I32, I32, P, P, P]),
    "cubic_merge_prefix": (I32, [P, I32, I32, P, I32, P, P]),
    "cubic_greedy_workspace_bytes": (I64, [I32, I32]),
    "cubic_greedy_candidates": (I32, [P, I32, I64, I32, I32, I64, P, P, I64, P, I64, I32, P, P, P, I64, P]),
    "cubic_greedy_root": (I32, [P, I32, P, P, P, P, P, P, P, I32, I32, I32, I64, P, P, P]),
    "cubic_sampling_final_guard": (I32, [P, P, P, P, P, P, P, P, I32, I32, I64, P, P]),
    "cubic_greedy_sample": (I32, [P, I32, I64, I32, I32, P, P, I64, P, I64, I32, P, P, P, P, P, I64, P,
                                  P, P, P, P, P, I64, P]),
    "cubic_accept_workspace_bytes": (I64, [I32, I32, I32]),
    "cubic_accept": (I32, [P, I64, I32, I32, I32, I32, P, P, P, P, I32, P, P, P, P, P, P, P, P, P,
                           P, P, P, P, I64, P]),
    "cubic_accept_noalloc": (I32, [P, I64, I32, I32, I32, I32, P, P, P, P, I32, P, P, P, P, P, P, P,
                                   P, P, P, P, P, P]),
}


class NativeError(RuntimeError):
    """A C-ABI call returned a negative status."""

    def __init__(self, name: str, code: int, message: str):
        super().__init__(f"{name} failed ({code}): {message}")
        self.code = code


def library_path() -> Path:
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    """Load the HIP library; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise RuntimeError(
                f"Cubic MI355X HIP library missing at {_LIB_PATH}; run "
                "`python -m cubic_serve_amd.build` (hipcc --offload-arch=gfx950)")
        handle = ctypes.CDLL(str(_LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        if handle.cubic_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{_LIB_PATH} implements ABI {handle.cubic_abi_version()}, these "
                               f"bindings expect {ABI_VERSION}: rebuild the library")
        _lib = handle
    return _lib


def call(name: str, *args) -> int:
    """Call an int-status entry point; raise ValueError/RuntimeError on failure."""
    status = getattr(lib(), name)(*args)
    if status < 0:
        message = (lib().cubic_last_error() or b"").decode(errors="replace")
        if status in (-1, -2, -4):
            raise ValueError(f"{name}: {message}")
        raise NativeError(name, status, message)
    return status


def ptr(tensor) -> int | None:
    """Device address of a tensor (None for a missing optional operand)."""
    return None if tensor is None else tensor.data_ptr()


def stream_of(device) -> int:
    import torch

    return int(torch.cuda.current_stream(device).cuda_stream)
