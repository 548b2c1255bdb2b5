"""ctypes binding of `libhackathon_amd.so` (the C-ABI declared in
include/hackathon_amd.h).

The library is loaded from the package directory only; there is no fallback.
A missing or unloadable library raises `HipLibraryError`, so nothing on the
product path can silently run somewhere else.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libhackathon_amd.so"

c_int = ctypes.c_int
c_int64 = ctypes.c_int64
c_float = ctypes.c_float
c_void_p = ctypes.c_void_p
c_char_p = ctypes.c_char_p

# Status codes (common.h).
HK_OK = 0
HK_ERR_ARG = -1
HK_ERR_HIP = -2
HK_ERR_CAPACITY = -3
HK_ERR_STATE = -4


class HipLibraryError(RuntimeError):
    """The HIP extension is missing, failed to load, or a call failed."""


class CapacityError(HipLibraryError):
    """More rows or runs than the engine was created for."""


# name -> (restype, argtypes)
_SIGNATURES = {
    "hk_version": (c_int, []),
    "hk_last_error": (c_char_p, []),
    "hk_mlstm_step": (c_int, [c_void_p] * 8 + [c_int] * 4 + [c_void_p]),
    "hk_retnet_step": (c_int, [c_void_p] * 7 + [c_int] * 4 + [c_void_p]),
    "hk_mamba2_step": (c_int, [c_void_p] * 8 + [c_int] * 4 + [c_void_p]),
    "hk_conv1d_step": (c_int, [c_void_p] * 6 + [c_int] * 3 + [c_void_p]),
    "hk_block_linear": (c_int, [c_void_p] * 4 + [c_int] * 3 + [c_void_p]),
    "hk_rglru_step": (c_int, [c_void_p] * 5 + [c_float] + [c_void_p] * 2 + [c_int] * 2
                      + [c_void_p]),
    "hk_slstm_step": (c_int, [c_void_p] * 9 + [c_int] * 2 + [c_void_p]),
    "hk_pack_tick": (c_int, [c_void_p] * 2 + [c_int] + [c_void_p] * 6),
    "hk_cast_linear": (c_int, [c_void_p] * 4 + [c_int] * 4 + [c_void_p, c_int64, c_void_p]),
    "hk_pack_cast_weight": (c_int, [c_void_p] * 2 + [c_int] * 2 + [c_void_p]),
    "hk_cast_linear_packed": (c_int, [c_void_p] * 4 + [c_int] * 5 + [c_void_p, c_int64, c_void_p]),
}

_lib = None


def declared_symbols() -> list[str]:
    return sorted(_SIGNATURES)


def register(name: str, restype, argtypes) -> None:
    """Add a signature (used by modules that bind further entry points)."""
    _SIGNATURES[name] = (restype, argtypes)
    if _lib is not None:
        fn = getattr(_lib, name)
        fn.restype = restype
        fn.argtypes = argtypes


def lib():
    """The loaded library, with every declared signature bound."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise HipLibraryError(
                f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`"
            )
        try:
            handle = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:  # pragma: no cover - depends on the machine
            raise HipLibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status == HK_OK:
        return
    msg = lib().hk_last_error().decode(errors="replace")
    if status == HK_ERR_CAPACITY:
        raise CapacityError(f"{what}: {msg}")
    raise HipLibraryError(f"{what} failed ({status}): {msg}")


def ptr(t) -> int:
    """Device (or host) address of a torch tensor, or None for None."""
    return None if t is None else t.data_ptr()


def current_stream(device) -> int:
    import torch

    return torch.cuda.current_stream(device).cuda_stream
