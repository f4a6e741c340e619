"""ctypes binding of ``libfoldforge_amd.so`` (the C-ABI declared in ``include/foldforge_amd.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime torch already
loaded (both carry the soname ``libamdhip64.so.7``): device pointers and stream handles
are then shared with torch's allocator and streams. There is no fallback: a missing or
unloadable library raises :class:`NativeUnavailable`.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

LIBRARY = Path(__file__).resolve().with_name("libfoldforge_amd.so")

#: symbol -> (restype, argtypes); mirrors include/foldforge_amd.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "ffk_version": (c_int32, []),
    "ffk_last_error": (ctypes.c_char_p, []),
    "ffk_device_supported": (c_int32, [c_int32]),
    "ffk_layer_norm": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_float, c_int32, c_void_p],
    ),
    "ffk_triangle_multiplication_workspace": (c_size_t, [c_int64, c_int64, c_int32, c_int32]),
    "ffk_triangle_multiplication": (
        c_int32,
        [c_void_p] * 13
        + [c_void_p, c_size_t, c_int64, c_int64, c_int32, c_int32, c_int32, c_int32, c_int32,
           c_float, c_void_p],
    ),
    "ffk_triangle_attention_workspace": (
        c_size_t,
        [c_int64, c_int64, c_int32, c_int32, c_int32, c_int32],
    ),
    "ffk_triangle_attention": (
        c_int32,
        [c_void_p] * 15
        + [c_void_p, c_size_t, c_int64, c_int64, c_int32, c_int32, c_int32, c_int32, c_int32,
           c_int32, c_int32, c_float, c_void_p],
    ),
    "ffk_triangle_attention_transition_workspace": (c_size_t, [c_int64, c_int64]),
    "ffk_triangle_attention_transition": (
        c_int32,
        [c_void_p] * 16 + [c_void_p, c_size_t, c_int64, c_int64, c_int32, c_int32, c_float,
                           c_float, c_void_p],
    ),
    "ffk_flash_attention_bias": (
        c_int32,
        [c_void_p] * 5
        + [c_int64, c_int32, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,
           c_void_p],
    ),
    "ffk_transition_workspace": (c_size_t, [c_int64, c_int32, c_int32]),
    "ffk_transition": (
        c_int32,
        [c_void_p] * 7
        + [c_void_p, c_size_t, c_int64, c_int32, c_int32, c_int32, c_float, c_void_p],
    ),
    "ffk_transition_noalloc": (
        c_int32,
        [c_void_p] * 7 + [c_int64, c_int32, c_int32, c_int32, c_float, c_void_p],
    ),
    "ffk_layer_norm_linear": (
        c_int32,
        [c_void_p] * 6 + [c_int64, c_int32, c_int32, c_int32, c_int32, c_float, c_void_p],
    ),
    "ffk_swiglu_ffn_workspace": (c_size_t, [c_int64, c_int32]),
    "ffk_swiglu_ffn": (
        c_int32,
        [c_void_p] * 7 + [c_size_t, c_int64, c_int32, c_int32, c_void_p],
    ),
    "ffk_msa_pair_weighted_averaging_workspace": (
        c_size_t,
        [c_int64, c_int64, c_int64, c_int32, c_int32, c_int32, c_int32],
    ),
    "ffk_msa_pair_weighted_averaging": (
        c_int32,
        [c_void_p] * 12
        + [c_size_t, c_int64, c_int64, c_int64, c_int32, c_int32, c_int32, c_int32, c_int32,
           c_float, c_float, c_void_p],
    ),
    "ffk_outer_product_mean_workspace": (
        c_size_t,
        [c_int64, c_int64, c_int64, c_int32, c_int32, c_int32],
    ),
    "ffk_outer_product_mean": (
        c_int32,
        [c_void_p] * 13
        + [c_size_t, c_int64, c_int64, c_int64, c_int32, c_int32, c_int32, c_float, c_float,
           c_int32, c_void_p],
    ),
    "ffk_outer_product_mean_grouped_workspace": (
        c_size_t,
        [c_int64, c_int64, c_int64, c_int32, c_int32, c_int32, c_int32],
    ),
    "ffk_outer_product_mean_grouped": (
        c_int32,
        [c_void_p] * 15
        + [c_size_t, c_int64, c_int64, c_int64, c_int32, c_int32, c_int32, c_int32, c_float, c_float,
           c_void_p],
    ),
    "ffk_attention_pair_bias_workspace": (
        c_size_t,
        [c_int64, c_int64, c_int32, c_int32, c_int32],
    ),
    "ffk_attention_pair_bias": (
        c_int32,
        [c_void_p] * 13
        + [c_void_p, c_int32, c_int64, c_int64, c_int64, c_void_p, c_void_p]
        + [c_size_t, c_int64, c_int64, c_int32, c_int32, c_int32, c_float, c_int32, c_float,
           c_float, c_void_p],
    ),
}


class NativeUnavailable(RuntimeError):
    """The HIP library is not built or cannot be loaded (there is no fallback path)."""


class NativeError(RuntimeError):
    """A non-zero status from the C-ABI (a kernel failure, not a backend refusal)."""


_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library with every declared symbol typed (loads it on first use)."""
    global _lib
    if _lib is None:
        import torch  # noqa: F401  - binds the library to torch's HIP runtime

        if not LIBRARY.exists():
            raise NativeUnavailable(
                f"{LIBRARY} is not built; run `python -m foldforge_amd.build` "
                "(the hip backend has no fallback)"
            )
        try:
            handle = ctypes.CDLL(str(LIBRARY))
        except OSError as exc:
            raise NativeUnavailable(f"cannot load {LIBRARY}: {exc}") from exc
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    """Raise :class:`NativeError` with the library's message for a non-zero status."""
    if status != 0:
        message = lib().ffk_last_error().decode(errors="replace")
        raise NativeError(f"{what}: {message} (status {status})")
