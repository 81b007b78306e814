"""The private seam between the public descriptor and the HIP plugin.

``HipBackend`` plays the role of the reference's ``CudaBackend``
(``src/mdescriptor/core/backends.py:86-290``): construction only stores the
validated options, and the plugin (``mdescriptor_amd._hip``) is loaded, the
device selected and the plan uploaded on the first ``compute``.  Errors from
the plugin are mapped onto the public error schema (``errors.py:83-145``).

Batches are submitted in blocks of whole structures bounded by an atom
budget rather than the reference's fixed 32 structures (``backends.py:
192-249``): a batch of many small molecules then needs one device round trip
instead of hundreds, while a cancellation still takes effect at the next
block boundary (and, inside a block, between kernel launches).  Every block
writes its rows straight into one preallocated output matrix.
"""

from __future__ import annotations

from collections.abc import Iterator, Mapping
from contextlib import contextmanager
from typing import Any

import numpy as np

from .. import _hip
from .errors import CancelledError, MDescriptorError, translate_backend_error

# Atoms per device submission.  A block's graph, coefficients and output
# staging live in HBM together; 2^20 atoms keep that far below one GPU's
# memory at every supported (species, n_max, l_max).
ATOM_BUDGET = 1 << 20


def structure_blocks(offsets: np.ndarray, budget: int = ATOM_BUDGET) -> list[tuple[int, int]]:
    """Split structures ``[0, S)`` into consecutive ``[start, stop)`` ranges of
    at most ``budget`` atoms each; a structure larger than the budget gets a
    block of its own.  An empty batch gives no blocks."""

    offsets = np.asarray(offsets, dtype=np.int64)
    structures = len(offsets) - 1
    blocks: list[tuple[int, int]] = []
    start = 0
    while start < structures:
        limit = offsets[start] + budget
        stop = int(np.searchsorted(offsets, limit, side="right")) - 1
        stop = min(max(stop, start + 1), structures)
        blocks.append((start, stop))
        start = stop
    return blocks


@contextmanager
def _plugin_errors() -> Iterator[None]:
    """Map plugin failures onto the public error schema (errors.py:83-145)."""

    try:
        yield
    except MDescriptorError:
        raise
    except Exception as exc:
        if isinstance(exc, _hip.HipCancelledError):
            raise CancelledError("descriptor computation was cancelled") from exc
        if isinstance(exc, ValueError):
            raise
        raise translate_backend_error(exc, unavailable_message="HIP backend is unavailable",
                                      failure_message="HIP backend failed") from exc


class HipBackend:
    """Lazy proxy for the HIP plugin.  ``level="pair"`` selects the pair-level
    contract (NeighborList): per-block results are concatenated, since the
    row count is known only after the device has filtered the pairs."""

    def __init__(self, name: str, options: Mapping[str, Any], feature_count: int | None = None,
                 atom_budget: int = ATOM_BUDGET, level: str | None = None) -> None:
        self.name = name
        self.options = dict(options)
        self._feature_count = feature_count
        self._implementation: Any = None
        self._closed = False
        self.atom_budget = int(atom_budget)
        self.level = level
        self.last_timing: dict[str, float] = {}

    @property
    def feature_count(self) -> int | None:
        return self._feature_count

    def _ensure_implementation(self) -> Any:
        if self._closed:
            raise RuntimeError("HIP backend is closed")
        if self._implementation is None:
            from .._runtime import create_hip_backend

            self._implementation = create_hip_backend(self.name, self.options)
            self._feature_count = int(self._implementation.feature_count)
        return self._implementation

    def compute(self, batch: Any, control: Any = None) -> dict[str, Any]:
        implementation = self._ensure_implementation()
        if self.level == "pair":
            return self._compute_pairs(implementation, batch, control)
        average = str(self.options.get("average", "inner"))
        dtype = np.dtype((self.options.get("output") or {}).get("dtype", "float64"))
        level = "atom" if average == "off" else "structure"
        rows = batch.atoms if level == "atom" else batch.structures
        values = _hip.pinned_empty((rows, int(self._feature_count)), dtype)
        blocks = structure_blocks(batch.offsets, self.atom_budget)
        if control is not None:
            control.reset(batch.structures)
        timing: dict[str, float] = {}
        with _plugin_errors():
            for start, stop in blocks:
                if control is not None and control.cancelled():
                    raise CancelledError("descriptor computation was cancelled")
                block = batch if (start, stop) == (0, batch.structures) else batch._slice_view(start, stop)
                if level == "atom":
                    target = values[int(batch.offsets[start]):int(batch.offsets[stop])]
                else:
                    target = values[start:stop]
                raw = implementation.compute(block, control, out=target)
                for key, value in getattr(implementation, "last_timing", {}).items():
                    timing[key] = timing.get(key, 0.0) + float(value)
                del raw
                if control is not None:
                    for _ in range(stop - start):
                        control.mark_completed()
        self.last_timing = timing
        result: dict[str, Any] = {
            "values": values,
            "level": level,
            "labels": tuple(self.options.get("_hip_labels") or ()),
            "metadata": implementation.metadata(),
        }
        if level == "atom":
            result["row_offsets"] = np.asarray(batch.offsets, dtype=np.int64).copy()
        return result

    def compute_into(self, batch: Any, address: int, pitch: int, control: Any = None) -> None:
        """Write the rows of every block straight into a caller's device
        matrix (``pitch`` bytes per row) through the device-resident path."""

        implementation = self._ensure_implementation()
        average = str(self.options.get("average", "inner"))
        if control is not None:
            control.reset(batch.structures)
        with _plugin_errors():
            for start, stop in structure_blocks(batch.offsets, self.atom_budget):
                if control is not None and control.cancelled():
                    raise CancelledError("descriptor computation was cancelled")
                block = batch if (start, stop) == (0, batch.structures) else batch._slice_view(start, stop)
                first_row = int(batch.offsets[start]) if average == "off" else start
                implementation.compute_into(block, address + first_row * pitch, pitch, control)
                if control is not None:
                    for _ in range(stop - start):
                        control.mark_completed()

    def _compute_pairs(self, implementation: Any, batch: Any, control: Any) -> dict[str, Any]:
        """Pair-level rows of every block, in structure order; block samples
        count structures from the block's first one and are shifted here,
        as the reference shifts its chunks' pair records (backends.py:230-241,
        460-462)."""

        width = int(self._feature_count or 0)
        if control is not None:
            control.reset(batch.structures)
        parts: list[dict[str, Any]] = []
        starts: list[int] = []
        with _plugin_errors():
            for start, stop in structure_blocks(batch.offsets, self.atom_budget):
                if control is not None and control.cancelled():
                    raise CancelledError("descriptor computation was cancelled")
                block = batch if (start, stop) == (0, batch.structures) else batch._slice_view(start, stop)
                parts.append(implementation.compute(block, control))
                starts.append(start)
                if control is not None:
                    for _ in range(stop - start):
                        control.mark_completed()
        if len(parts) == 1:
            values, samples, row_offsets = parts[0]["values"], parts[0]["samples"], parts[0]["row_offsets"]
        else:
            values = np.concatenate([p["values"] for p in parts]) if parts else np.empty((0, width))
            shifted = []
            for part, start in zip(parts, starts):
                block_samples = np.array(part["samples"], dtype=np.int64, copy=True)
                block_samples[:, 0] += start
                shifted.append(block_samples)
            samples = np.concatenate(shifted) if shifted else np.empty((0, 6), dtype=np.int64)
            row_offsets = np.zeros(batch.structures + 1, dtype=np.int64)
            for part, start in zip(parts, starts):
                local = np.asarray(part["row_offsets"], dtype=np.int64)
                row_offsets[start + 1:start + len(local)] = local[1:] + row_offsets[start]
        return {
            "values": values,
            "level": "pair",
            "labels": tuple(getattr(implementation, "labels", ()) or ()),
            "row_offsets": np.asarray(row_offsets, dtype=np.int64),
            "samples": samples,
            "metadata": implementation.metadata(),
        }

    def metadata(self) -> Mapping[str, Any]:
        if self._implementation is None:
            return {"descriptor": self.name, "backend": "mdescriptor-hip"}
        return self._implementation.metadata()

    def close(self) -> None:
        if self._implementation is not None:
            self._implementation.close()
        self._implementation = None
        self._closed = True


__all__ = ["ATOM_BUDGET", "HipBackend", "structure_blocks"]
