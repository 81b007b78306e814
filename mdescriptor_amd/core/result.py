"""Descriptor results and their sample indices.

Follows ``src/mdescriptor/core/result.py``: :func:`format_values` (``:64-87``)
is the single dense/CSR representation rule, ``atom_samples`` /
``structure_samples`` (``:234-260``) give each row its identity, and
:class:`DescriptorResult` (``:306-420``) validates values, labels, offsets and
samples together and stores read-only snapshots.  Fresh arrays produced by
the HIP backend are handed over with :class:`_OwnedValues` so a
gigabyte-sized matrix is not copied a second time on its way out.
"""

from __future__ import annotations

import json
import math
from collections.abc import Mapping
from copy import copy, deepcopy
from dataclasses import dataclass, field
from enum import Enum
from typing import Any

import numpy as np

from .errors import DescriptorConfigError

RESULT_SCHEMA_VERSION = 1


class DescriptorLevel(str, Enum):
    ATOM = "atom"
    STRUCTURE = "structure"
    PAIR = "pair"


class _OwnedValues:
    """A fresh C-contiguous matrix that the result may keep without copying:
    either an array owning its memory or a whole page-locked block from the
    HIP plugin's pool (an array whose base is the block's owner)."""

    __slots__ = ("array",)

    def __init__(self, array: Any) -> None:
        if not isinstance(array, np.ndarray):
            raise TypeError("owned descriptor values must be a NumPy array")
        owner = array.flags.owndata or (array.base is not None and not isinstance(array.base, np.ndarray)
                                        and hasattr(array.base, "__array_interface__"))
        if array.ndim != 2 or not array.flags.c_contiguous or not owner:
            raise ValueError("owned descriptor values must be a C-contiguous owning matrix")
        array.setflags(write=False)
        self.array = array


def owned_values(array: np.ndarray) -> _OwnedValues:
    return _OwnedValues(array)


def format_values(values: Any, *, dtype: str = "float64", sparse: bool = False) -> Any:
    """Dense array of ``dtype`` or, with ``sparse``, a CSR matrix (result.py:64-87)."""

    target = np.dtype(dtype)
    try:
        import scipy.sparse as scipy_sparse
    except ImportError:  # pragma: no cover - scipy is a dependency of this image
        scipy_sparse = None
    if sparse:
        if scipy_sparse is None:  # pragma: no cover
            raise DescriptorConfigError("sparse output requires scipy")
        if scipy_sparse.issparse(values):
            return values.tocsr().astype(target, copy=False)
        return scipy_sparse.csr_matrix(np.asarray(values, dtype=target))
    if scipy_sparse is not None and scipy_sparse.issparse(values):
        return np.asarray(values.toarray(), dtype=target)
    return np.asarray(values, dtype=target)


def structure_samples(rows: int) -> np.ndarray:
    """``[structure]`` sample per structure-level row (result.py:234-237)."""

    return np.arange(rows, dtype=np.int64).reshape(rows, 1)


def atom_samples(row_offsets: np.ndarray) -> np.ndarray:
    """``[structure, local_atom]`` sample per atom-level row (result.py:240-255)."""

    offsets = np.ascontiguousarray(row_offsets, dtype=np.int64)
    if offsets.ndim != 1 or len(offsets) == 0:
        raise ValueError("atom row offsets must be a non-empty one-dimensional array")
    counts = np.diff(offsets)
    structure = np.repeat(np.arange(len(counts), dtype=np.int64), counts)
    local = np.arange(int(offsets[-1] - offsets[0]), dtype=np.int64) - np.repeat(offsets[:-1] - offsets[0], counts)
    return np.column_stack((structure, local)).astype(np.int64, copy=False)


def _snapshot_values(values: Any) -> Any:
    if isinstance(values, _OwnedValues):
        return values.array
    try:
        import scipy.sparse as scipy_sparse
    except ImportError:  # pragma: no cover
        scipy_sparse = None
    if scipy_sparse is not None and scipy_sparse.issparse(values):
        snapshot = values.tocsr(copy=True)
        snapshot.sum_duplicates()
        snapshot.sort_indices()
        for array in (snapshot.data, snapshot.indices, snapshot.indptr):
            array.setflags(write=False)
        return snapshot
    try:
        snapshot = np.array(values, copy=True, order="C")
    except (TypeError, ValueError, OverflowError) as exc:
        raise ValueError("descriptor values must be a two-dimensional array") from exc
    if snapshot.ndim != 2:
        raise ValueError("descriptor values must be a two-dimensional array")
    snapshot.setflags(write=False)
    return snapshot


def _json_safe(value: Any) -> Any:
    if isinstance(value, Mapping):
        return {str(k): _json_safe(v) for k, v in value.items()}
    if isinstance(value, (list, tuple)):
        return [_json_safe(v) for v in value]
    if isinstance(value, np.ndarray):
        return _json_safe(value.tolist())
    if isinstance(value, np.generic):
        return _json_safe(value.item())
    if isinstance(value, float) and not math.isfinite(value):
        raise TypeError("metadata cannot contain non-finite numbers")
    if value is None or isinstance(value, (str, int, float, bool)):
        return value
    to_dict = getattr(value, "to_dict", None)
    if callable(to_dict):
        return _json_safe(to_dict())
    raise TypeError(f"metadata value is not JSON-safe: {type(value).__name__}")


def metadata_envelope(raw: Mapping[str, Any], level: str, feature_count: int | None) -> dict[str, Any]:
    """The fixed metadata envelope of a result (result.py:504-560): descriptor,
    backend, output, execution, level, feature_count and, when there are
    any, the backend ``details``."""

    data = _json_safe(dict(raw))
    descriptor = data.pop("descriptor", "unknown")
    backend = data.pop("backend", "unknown")
    for key in ("schema_version", "level", "feature_count"):
        data.pop(key, None)
    details = data.pop("details", None)
    flat_output = {"dtype": data.pop("dtype", "float64"), "sparse": data.pop("sparse", False)}
    flat_execution = {"device": data.pop("device", "hip"), "num_threads": data.pop("num_threads", None)}
    output = data.pop("output", None) or flat_output
    execution = data.pop("execution", None) or flat_execution
    data.pop("pair_records", None)  # pair identity lives in the samples only
    merged = dict(details or {})
    merged.update(data)
    envelope = {
        "schema_version": RESULT_SCHEMA_VERSION,
        "descriptor": descriptor,
        "backend": backend,
        "level": str(level),
        "feature_count": feature_count,
        "output": {"dtype": output.get("dtype", "float64"), "sparse": bool(output.get("sparse", False))},
        "execution": {"device": execution.get("device", "hip"), "num_threads": execution.get("num_threads")},
    }
    if merged:
        envelope["details"] = merged
    return envelope


@dataclass(frozen=True, slots=True)
class DescriptorResult:
    """Values plus row and feature identities, detached from kernel storage."""

    values: Any
    level: DescriptorLevel | str
    structure_ids: tuple[str, ...]
    row_offsets: np.ndarray | None
    labels: tuple[str, ...]
    metadata: Mapping[str, Any] = field(default_factory=dict)
    samples: Any = None
    feature_count: int | None = None
    # Atom offsets of the batch, needed to validate the local atom indices of
    # pair samples; construction context only, never serialised (result.py:320-327).
    _atom_row_offsets: np.ndarray | None = field(default=None, repr=False, compare=False, kw_only=True)

    def __post_init__(self) -> None:
        level = DescriptorLevel(self.level)
        object.__setattr__(self, "level", level)
        object.__setattr__(self, "structure_ids", tuple(str(v) for v in self.structure_ids))
        labels = tuple(str(v) for v in self.labels)
        object.__setattr__(self, "labels", labels)
        values = _snapshot_values(self.values)
        object.__setattr__(self, "values", values)
        rows, width = int(values.shape[0]), int(values.shape[1])
        if len(labels) != width:
            raise ValueError("labels must contain exactly one entry per feature column")
        count = width if self.feature_count is None else self.feature_count
        if isinstance(count, bool) or int(count) != width:
            raise ValueError("feature_count does not match the result feature dimension")
        object.__setattr__(self, "feature_count", int(count))

        offsets = self.row_offsets
        if offsets is not None:
            raw = np.asarray(offsets)
            if raw.ndim != 1 or not np.issubdtype(raw.dtype, np.integer):
                raise ValueError("row offsets must be a one-dimensional integer array")
            offsets = np.array(raw, dtype=np.int64, order="C", copy=True)
            offsets.setflags(write=False)
            object.__setattr__(self, "row_offsets", offsets)
        if level is DescriptorLevel.STRUCTURE:
            if offsets is not None:
                raise ValueError("structure-level results cannot have row offsets")
            if rows != len(self.structure_ids):
                raise ValueError("structure-level results need one row per structure")
        else:
            if offsets is None:
                raise ValueError(f"{level.value}-level results require row offsets")
            if len(offsets) != len(self.structure_ids) + 1 or offsets[0] != 0 or int(offsets[-1]) != rows:
                raise ValueError(f"{level.value} row offsets must cover every row, one entry per structure boundary")
            if np.any(np.diff(offsets) < 0):
                raise ValueError(f"{level.value} row offsets must be non-decreasing")
        atom_offsets = self._atom_row_offsets
        if atom_offsets is not None:
            raw = np.asarray(atom_offsets)
            if raw.ndim != 1 or not np.issubdtype(raw.dtype, np.integer):
                raise ValueError("atom row offsets must be a one-dimensional integer array")
            atom_offsets = np.array(raw, dtype=np.int64, order="C", copy=True)
            if len(atom_offsets) != len(self.structure_ids) + 1 or atom_offsets[0] != 0:
                raise ValueError("atom row offsets must start at zero, one entry per structure boundary")
            if np.any(np.diff(atom_offsets) < 0):
                raise ValueError("atom row offsets must be non-decreasing")
            atom_offsets.setflags(write=False)
            object.__setattr__(self, "_atom_row_offsets", atom_offsets)

        samples = self.samples
        if samples is None:
            if level is DescriptorLevel.STRUCTURE:
                samples = structure_samples(rows)
            elif level is DescriptorLevel.ATOM:
                samples = atom_samples(offsets)
            else:
                raise ValueError("pair-level results require explicit pair samples")
        samples = np.asarray(samples)
        if samples.size and not np.issubdtype(samples.dtype, np.integer):
            raise ValueError("samples must contain integer indices")
        samples = np.array(samples, dtype=np.int64, order="C", copy=True)
        expected = {DescriptorLevel.STRUCTURE: 1, DescriptorLevel.ATOM: 2, DescriptorLevel.PAIR: 6}[level]
        if samples.ndim != 2 or samples.shape != (rows, expected):
            raise ValueError(f"{level.value}-level samples must have shape (rows, {expected})")
        if level is DescriptorLevel.PAIR:
            # result.py:399-410: structure and both local atom indices in range
            if atom_offsets is None:
                raise ValueError("pair-level results require atom row offsets for sample validation")
            if rows and (np.any(samples[:, :3] < 0) or np.any(samples[:, 0] >= len(offsets) - 1)):
                raise ValueError("pair samples contain an invalid structure or atom index")
            counts = np.diff(atom_offsets)
            if rows and (np.any(samples[:, 1] >= counts[samples[:, 0]])
                         or np.any(samples[:, 2] >= counts[samples[:, 0]])):
                raise ValueError("pair samples contain an invalid local atom index")
        samples.setflags(write=False)
        object.__setattr__(self, "samples", samples)
        object.__setattr__(self, "metadata", json.loads(json.dumps(_json_safe(self.metadata))))

    @property
    def rows(self) -> int:
        return int(self.values.shape[0])

    def _replace_output(self, values: Any, output: Mapping[str, Any]) -> DescriptorResult:
        """Same result with values re-represented and ``metadata.output`` updated."""

        metadata = deepcopy(dict(self.metadata))
        metadata["output"] = dict(output)
        updated = copy(self)
        object.__setattr__(updated, "values", _snapshot_values(values))
        object.__setattr__(updated, "metadata", metadata)
        return updated

    def to_dict(self) -> dict[str, Any]:
        """JSON-safe result without the values matrix."""

        return {
            "level": self.level.value,
            "structure_ids": list(self.structure_ids),
            "row_offsets": None if self.row_offsets is None else self.row_offsets.tolist(),
            "labels": list(self.labels),
            "feature_count": self.feature_count,
            "samples": self.samples.tolist(),
            "metadata": deepcopy(dict(self.metadata)),
        }


__all__ = [
    "DescriptorLevel",
    "DescriptorResult",
    "RESULT_SCHEMA_VERSION",
    "atom_samples",
    "format_values",
    "metadata_envelope",
    "owned_values",
    "structure_samples",
]
