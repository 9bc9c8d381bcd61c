"""ctypes binding of ``libbioemu2_mi355x.so`` (the C ABI in ``include/bioemu2_mi355x.h``).

The library is loaded lazily on first use.  There is no fallback: if the
library is missing or fails to load, every op raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libbioemu2_mi355x.so"

_c_void_p = ctypes.c_void_p
_c_size_t = ctypes.c_size_t
_c_int64 = ctypes.c_int64
_c_int = ctypes.c_int

# name -> (restype, argtypes).  Keep in the order of include/bioemu2_mi355x.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "bioemu_version": (ctypes.c_char_p, []),
    "bioemu_last_error": (ctypes.c_char_p, []),
    "bioemu_timer_enable": (_c_int, [_c_int]),
    "bioemu_timer_reset": (_c_int, []),
    "bioemu_timer_count": (_c_int, []),
    "bioemu_timer_query": (
        _c_int,
        [_c_int, ctypes.c_char_p, _c_size_t, ctypes.POINTER(_c_int64), ctypes.POINTER(ctypes.c_double)],
    ),
    "bioemu_trimul_workspace_bytes": (_c_size_t, [_c_int64, _c_int64, _c_int64]),
    "bioemu_trimul_fwd": (
        _c_int,
        [_c_void_p] * 12 + [_c_void_p, _c_size_t, _c_int64, _c_int64, _c_int64, _c_int, _c_int, _c_void_p],
    ),
    "bioemu_triatt_workspace_bytes": (_c_size_t, [_c_int64] * 4),
    "bioemu_triatt_fwd": (
        _c_int,
        [_c_void_p] * 8 + [_c_void_p, _c_size_t] + [_c_int64] * 4 + [_c_int, _c_int, _c_void_p],
    ),
    "bioemu_transition_pair_workspace_bytes": (_c_size_t, [_c_int64] * 2),
    "bioemu_transition_pair_fwd": (
        _c_int,
        [_c_void_p] * 8 + [_c_void_p, _c_size_t] + [_c_int64] * 3 + [_c_int, _c_int, _c_void_p],
    ),
    "bioemu_transition_pair_fwd_noalloc": (
        _c_int,
        [_c_void_p] * 8 + [_c_int64] * 3 + [_c_int, _c_int, _c_void_p],
    ),
    "bioemu_transition_token_workspace_bytes": (_c_size_t, [_c_int64] * 3),
    "bioemu_transition_token_fwd": (
        _c_int,
        [_c_void_p] * 8 + [_c_void_p, _c_size_t] + [_c_int64] * 4 + [_c_int, _c_int, _c_void_p],
    ),
    "bioemu_pwa_workspace_bytes": (_c_size_t, [_c_int64] * 6),
    "bioemu_pwa_fwd": (
        _c_int,
        [_c_void_p] * 13 + [_c_void_p, _c_size_t] + [_c_int64] * 7 + [_c_int, _c_void_p],
    ),
    "bioemu_apb_workspace_bytes": (_c_size_t, [_c_int64] * 5),
    "bioemu_apb_fwd": (
        _c_int,
        [_c_void_p] * 14 + [_c_void_p, _c_size_t] + [_c_int64] * 6 + [_c_int, _c_void_p],
    ),
    "bioemu_swa_workspace_bytes": (_c_size_t, [_c_int64] * 7),
    "bioemu_swa_fwd": (
        _c_int,
        [_c_void_p] * 13 + [_c_void_p, _c_size_t] + [_c_int64] * 8 + [_c_int, _c_void_p],
    ),
    "bioemu_distogram_fwd": (_c_int, [_c_void_p] * 4 + [_c_int64] * 4 + [_c_int, _c_void_p]),
    "bioemu_pair_cond_workspace_bytes": (_c_size_t, [_c_int64] * 3),
    "bioemu_pair_cond_proj_fwd": (
        _c_int,
        [_c_void_p] * 8 + [_c_size_t] + [_c_int64] * 4 + [_c_void_p],
    ),
    "bioemu_opm_workspace_bytes": (_c_size_t, [_c_int64] * 5),
    "bioemu_opm_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_int] + [_c_void_p] * 9 + [_c_size_t] + [_c_int64] * 6 + [_c_void_p],
    ),
    "bioemu_stream_split": (_c_int, [_c_void_p] * 3 + [_c_int64, _c_void_p]),
    "bioemu_stream_join": (_c_int, [_c_void_p] * 3 + [_c_int64, _c_void_p]),
    "bioemu_pair_ln_linear_workspace_bytes": (_c_size_t, [_c_int64]),
    "bioemu_pair_ln_linear_fwd": (_c_int, [_c_void_p] * 9 + [_c_size_t, _c_int64, _c_int64, _c_void_p]),
    "bioemu_token_ln_linear_workspace_bytes": (_c_size_t, [_c_int64] * 2),
    "bioemu_token_ln_linear_fwd": (_c_int, [_c_void_p] * 9 + [_c_size_t, _c_int64, _c_int64, _c_void_p]),
    "bioemu_trunk_uncond_workspace_bytes": (_c_size_t, [_c_int64] * 3),
    "bioemu_trunk_uncond_fwd": (_c_int, [_c_void_p] * 12 + [_c_size_t] + [_c_int64] * 3 + [_c_void_p]),
    "bioemu_msa_embed_workspace_bytes": (_c_size_t, [_c_int64] * 2),
    "bioemu_msa_embed_fwd": (_c_int, [_c_void_p] * 10 + [_c_size_t] + [_c_int64] * 6 + [_c_void_p]),
    "bioemu_apb_f32_workspace_bytes": (_c_size_t, [_c_int64] * 5),
    "bioemu_apb_fwd_f32": (_c_int, [_c_void_p] * 14 + [_c_size_t] + [_c_int64] * 6 + [_c_int, _c_void_p]),
    "bioemu_swa_f32_workspace_bytes": (_c_size_t, [_c_int64] * 7),
    "bioemu_swa_fwd_f32": (_c_int, [_c_void_p] * 14 + [_c_size_t] + [_c_int64] * 8 + [_c_int, _c_void_p]),
    "bioemu_transition_f32_workspace_bytes": (_c_size_t, [_c_int64] * 3),
    "bioemu_transition_fwd_f32": (
        _c_int,
        [_c_void_p] * 8 + [_c_size_t] + [_c_int64] * 4 + [_c_int, _c_int, _c_void_p],
    ),
    "bioemu_pair_cond_f32_workspace_bytes": (_c_size_t, [_c_int64] * 3),
    "bioemu_pair_cond_proj_fwd_f32": (_c_int, [_c_void_p] * 7 + [_c_size_t] + [_c_int64] * 4 + [_c_void_p]),
    "bioemu_triatt_f32_workspace_bytes": (_c_size_t, [_c_int64] * 4),
    "bioemu_triatt_fwd_f32": (
        _c_int,
        [_c_void_p] * 8 + [_c_size_t] + [_c_int64] * 4 + [_c_int, _c_int, _c_void_p],
    ),
    "bioemu_trimul_f32_workspace_bytes": (_c_size_t, [_c_int64] * 3),
    "bioemu_trimul_fwd_f32": (
        _c_int,
        [_c_void_p] * 12 + [_c_size_t] + [_c_int64] * 3 + [_c_int, _c_int, _c_void_p],
    ),
    "bioemu_opm_f32_workspace_bytes": (_c_size_t, [_c_int64] * 5),
    "bioemu_opm_fwd_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_int] + [_c_void_p] * 8 + [_c_size_t] + [_c_int64] * 6 + [_c_void_p],
    ),
    "bioemu_pwa_f32_workspace_bytes": (_c_size_t, [_c_int64] * 6),
    "bioemu_pwa_fwd_f32": (
        _c_int,
        [_c_void_p] * 13 + [_c_size_t] + [_c_int64] * 7 + [ctypes.c_float, _c_int, _c_void_p],
    ),
    "bioemu_msa_embed_fwd_f32": (_c_int, [_c_void_p] * 9 + [_c_size_t] + [_c_int64] * 6 + [_c_void_p]),
    "bioemu_ln_linear_f32_workspace_bytes": (_c_size_t, [_c_int64] * 2),
    "bioemu_ln_linear_fwd_f32": (_c_int, [_c_void_p] * 7 + [_c_size_t] + [_c_int64] * 3 + [_c_void_p]),
    "bioemu_trunk_uncond_f32_workspace_bytes": (_c_size_t, [_c_int64] * 3),
    "bioemu_trunk_uncond_fwd_f32": (_c_int, [_c_void_p] * 10 + [_c_size_t] + [_c_int64] * 3 + [_c_void_p]),
    "bioemu_distogram_f32_workspace_bytes": (_c_size_t, [_c_int64] * 3),
    "bioemu_distogram_fwd_f32": (_c_int, [_c_void_p] * 5 + [_c_size_t] + [_c_int64] * 4 + [_c_void_p]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class NativeLibraryError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Returns the loaded native library, loading it on first use."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise NativeLibraryError(
                    f"bioemu2_amd native library not found at {LIB_PATH}; "
                    "build it with `python -m bioemu2_amd.build` (hipcc, gfx950)"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    """Raises on a non-zero C-ABI return code, mapping codes to Python exceptions."""
    if rc == 0:
        return
    msg = lib().bioemu_last_error().decode(errors="replace")
    if rc in (-1, -2):
        raise ValueError(f"{what}: {msg} (code {rc})")
    raise RuntimeError(f"{what}: {msg} (code {rc})")
