"""Per-kernel timing through the library's hipEvent kernel timer.

While a :class:`KernelTimer` is active, every kernel the native library
launches is bracketed by hipEvents recorded on its own launch stream, so the
durations are those of the kernels themselves, not of torch's current stream.
"""

from __future__ import annotations

import ctypes

from ._lib import check, lib


class KernelTimer:
    """Context manager: ``with KernelTimer() as t: ...; t.results()``."""

    def __enter__(self) -> "KernelTimer":
        check(lib().bioemu_timer_reset(), "bioemu_timer_reset")
        check(lib().bioemu_timer_enable(1), "bioemu_timer_enable")
        return self

    def __exit__(self, *exc) -> None:
        lib().bioemu_timer_enable(0)

    @staticmethod
    def results() -> dict[str, tuple[int, float]]:
        """{kernel name: (launches, total ms)}; synchronises on pending events."""
        out: dict[str, tuple[int, float]] = {}
        buf = ctypes.create_string_buffer(128)
        n = ctypes.c_int64()
        ms = ctypes.c_double()
        for i in range(lib().bioemu_timer_count()):
            check(lib().bioemu_timer_query(i, buf, 128, ctypes.byref(n), ctypes.byref(ms)), "bioemu_timer_query")
            if n.value:
                out[buf.value.decode()] = (n.value, ms.value)
        return out
