"""Cooperative cancellation and progress (``src/mdescriptor/core/control.py:8-88``).

The public methods are the reference's.  The HIP backend also reads
``_hip_cancel_flag``: a ``ctypes.c_int32`` whose address is handed to the
C-ABI, which polls it between kernel launches and returns ``MDX_CANCELLED``
once :meth:`ComputeControl.cancel` has set it.
"""

from __future__ import annotations

import ctypes
import threading


class ComputeControl:
    """Cancellation flag plus a completed/total progress counter."""

    def __init__(self) -> None:
        self._lock = threading.Lock()
        self._hip_cancel_flag = ctypes.c_int32(0)
        self._completed = 0
        self._total = 0

    def reset(self, total: int) -> None:
        if isinstance(total, bool) or not isinstance(total, int) or total < 0:
            raise ValueError("control total must be a non-negative integer")
        with self._lock:
            self._hip_cancel_flag.value = 0
            self._completed = 0
            self._total = total

    def cancel(self) -> None:
        self._hip_cancel_flag.value = 1

    def cancelled(self) -> bool:
        return self._hip_cancel_flag.value != 0

    def completed(self) -> int:
        return self._completed

    def total(self) -> int:
        return self._total

    def mark_completed(self) -> None:
        with self._lock:
            self._completed += 1


__all__ = ["ComputeControl"]
