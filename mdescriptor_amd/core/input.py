"""The validated structure batch at the public seam.

``StructureBatch`` keeps the reference's value-object contract
(``src/mdescriptor/core/input.py:19-125``): five flattened arrays plus ids,
copied and validated on construction, read-only afterwards.  Fully periodic
structures carry a nonsingular cell and ``pbc = (1, 1, 1)``; isolated ones
``pbc = (0, 0, 0)`` and may carry a zero cell; mixed periodicity inside one
structure is rejected.  ``from_frames`` packs mapping/object frames;
``from_ase`` needs ASE, which is optional.
"""

from __future__ import annotations

from collections.abc import Iterable, Mapping, Sequence
from dataclasses import dataclass
from typing import Any

import numpy as np

from .errors import _InputValidationError


@dataclass(frozen=True)
class StructureBatch:
    """An owned, read-only snapshot of periodic or isolated structures."""

    numbers: np.ndarray
    positions: np.ndarray
    cells: np.ndarray
    pbc: np.ndarray
    offsets: np.ndarray
    ids: tuple[str, ...]
    spins: np.ndarray | None = None
    charge_spin: np.ndarray | None = None

    def __post_init__(self) -> None:
        numbers = _owned_array(self.numbers, np.int32, "numbers")
        positions = _owned_array(self.positions, np.float64, "positions")
        cells = _owned_array(self.cells, np.float64, "cells")
        pbc = _owned_array(self.pbc, np.int32, "pbc", allow_bool=True)
        offsets = _owned_array(self.offsets, np.int64, "offsets")
        ids = tuple(str(value) for value in self.ids)
        spins = None if self.spins is None else _owned_array(self.spins, np.float64, "spins")
        charge_spin = None if self.charge_spin is None else _owned_array(self.charge_spin, np.float64,
                                                                          "charge_spin")
        if numbers.ndim != 1 or np.any(numbers <= 0):
            raise _input_error("numbers must be a one-dimensional array of positive atomic numbers", "numbers")
        if positions.shape != (len(numbers), 3):
            raise _input_error("positions must have shape (total_atoms, 3)", "positions")
        if cells.ndim != 3 or cells.shape[1:] != (3, 3):
            raise _input_error("cells must have shape (structures, 3, 3)", "cells")
        if pbc.ndim != 2 or pbc.shape[1:] != (3,):
            raise _input_error("pbc must have shape (structures, 3)", "pbc")
        if offsets.ndim != 1 or len(offsets) != len(ids) + 1:
            raise _input_error("offsets must have one entry per structure plus a sentinel", "offsets")
        if len(cells) != len(ids) or len(pbc) != len(ids):
            raise _input_error("structure arrays and ids have inconsistent lengths", "structures")
        if len(offsets) and (offsets[0] != 0 or offsets[-1] != len(numbers)):
            raise _input_error("offsets must start at zero and end at total_atoms", "offsets")
        if np.any(offsets[1:] < offsets[:-1]):
            raise _input_error("offsets must be monotonic", "offsets")
        if np.any((pbc != 0) & (pbc != 1)):
            raise _input_error("pbc must contain only 0 or 1", "pbc")
        for index, matrix in enumerate(cells):
            flags = pbc[index]
            if bool(np.all(flags == 1)):
                if abs(float(np.linalg.det(matrix))) < 1e-14:
                    raise _input_error("periodic cells must be nonsingular", "cells")
            elif not bool(np.all(flags == 0)):
                raise _input_error("mixed periodicity is not supported; use all-zero or all-one pbc", "pbc")
        if spins is not None and spins.shape != (len(numbers), 3):
            raise _input_error("spins must have shape (total_atoms, 3)", "spins")
        if charge_spin is not None and charge_spin.shape != (len(ids), 2):
            raise _input_error("charge_spin must have shape (structures, 2)", "charge_spin")
        _install(self, dict(numbers=numbers, positions=positions, cells=cells, pbc=pbc, offsets=offsets, ids=ids,
                            spins=spins, charge_spin=charge_spin))

    @property
    def structures(self) -> int:
        return len(self.ids)

    @property
    def atoms(self) -> int:
        return len(self.numbers)

    def _slice_view(self, start: int, stop: int) -> StructureBatch:
        """Structures [start, stop) of this validated batch as a read-only
        batch sharing its arrays (no copy, no second validation)."""

        if not 0 <= start <= stop <= self.structures:
            raise ValueError("structure slice is outside the batch")
        first_atom, end_atom = (int(self.offsets[i]) for i in (start, stop))
        parts = {**{name: slice(first_atom, end_atom) for name in _PER_ATOM},
                 **{name: slice(start, stop) for name in _PER_STRUCTURE}}
        fields = {name: None if getattr(self, name) is None else getattr(self, name)[part]
                  for name, part in parts.items()}
        fields["offsets"] = (self.offsets[start:stop + 1] - first_atom).astype(np.int64)
        view = object.__new__(StructureBatch)
        _install(view, fields)
        return view

    @classmethod
    def from_frames(cls, frames: Iterable[Any] | Any) -> StructureBatch:
        """Pack frame records (mappings or objects with ``numbers``,
        ``positions``, ``cell``, ``pbc`` and ``id``) into one batch."""

        if isinstance(frames, Mapping) or not isinstance(frames, Iterable):
            values = [frames]
        else:
            values = list(frames)
        numbers, positions, cells, pbc, ids = [], [], [], [], []
        for index, frame in enumerate(values):
            numbers.append(np.asarray(_field(frame, ("numbers",), index)))
            positions.append(np.asarray(_field(frame, ("positions",), index)))
            cells.append(np.asarray(_field(frame, ("cell", "cells"), index)))
            pbc.append(np.asarray(_field(frame, ("pbc",), index)))
            ids.append(_field(frame, ("id",), index))
        offsets = np.concatenate([[0], np.cumsum([len(n) for n in numbers])]).astype(np.int64)
        return cls(
            np.concatenate(numbers) if numbers else np.empty(0, dtype=np.int32),
            np.concatenate(positions, axis=0) if positions else np.empty((0, 3)),
            np.stack(cells) if cells else np.empty((0, 3, 3)),
            np.stack(pbc) if pbc else np.empty((0, 3), dtype=np.int32),
            offsets,
            tuple(ids),
        )

    @classmethod
    def from_ase(cls, structures: Sequence[Any] | Any, ids: Sequence[str] | None = None) -> StructureBatch:
        try:
            from ase import Atoms
        except ImportError as exc:  # pragma: no cover - ASE is optional
            raise ImportError("ASE is required to build a StructureBatch from Atoms") from exc
        items = [structures] if isinstance(structures, Atoms) else list(structures)
        if ids is not None and len(ids) != len(items):
            raise _input_error("ids must have one entry per structure", "ids")
        frames = [
            {
                "numbers": atoms.get_atomic_numbers(),
                "positions": atoms.get_positions(),
                "cell": atoms.cell.array,
                "pbc": atoms.get_pbc().astype(np.int32),
                "id": str(ids[i]) if ids is not None else str(i),
            }
            for i, atoms in enumerate(items)
        ]
        return cls.from_frames(frames)


def coerce_batch(value: Any) -> StructureBatch:
    """Return an existing batch unchanged or pack ASE structures once."""

    if isinstance(value, StructureBatch):
        return value
    return StructureBatch.from_ase(value)


def _field(frame: Any, names: tuple[str, ...], index: int) -> Any:
    for name in names:
        if isinstance(frame, Mapping):
            if name in frame:
                return frame[name]
        elif hasattr(frame, name):
            return getattr(frame, name)
    raise _input_error(f"frame {index} is missing required field {names[0]!r}",
                       {"cell": "cells", "id": "ids"}.get(names[0], names[0]))


# fields indexed by atom and by structure, for cutting a batch into
# structure ranges (offsets are rebased separately)
_PER_ATOM = ("numbers", "positions", "spins")
_PER_STRUCTURE = ("cells", "pbc", "ids", "charge_spin")


def _install(batch: StructureBatch, fields: dict[str, Any]) -> None:
    """Set the fields of a frozen batch; its arrays become read-only."""

    for name, value in fields.items():
        if isinstance(value, np.ndarray):
            value.setflags(write=False)
        object.__setattr__(batch, name, value)


def _owned_array(value: Any, dtype: Any, field: str, *, allow_bool: bool = False) -> np.ndarray:
    """A private C-ordered copy of ``value`` as ``dtype``.

    Floating fields must convert and be finite.  Integer fields accept
    integer arrays, floats that are exact finite integers, and booleans
    where ``allow_bool`` (pbc); the values must fit ``dtype``."""

    if not np.issubdtype(dtype, np.integer):
        try:
            real = np.asarray(value, dtype=dtype)
        except (TypeError, ValueError, OverflowError) as exc:
            raise _input_error(f"{field} must be a numeric array", field) from exc
        if not np.all(np.isfinite(real)):
            raise _input_error(f"{field} must be finite", field)
        return np.array(real, dtype=dtype, order="C", copy=True)
    try:
        source = np.asarray(value)
    except (TypeError, ValueError, OverflowError) as exc:
        raise _input_error(f"{field} must be an integer array", field) from exc
    kind = source.dtype.kind
    if kind == "b" and not allow_bool:
        raise _input_error(f"{field} must contain integers, not booleans", field)
    if kind == "f" and not (np.all(np.isfinite(source)) and np.all(source == np.trunc(source))):
        raise _input_error(f"{field} must contain finite integers", field)
    if kind not in "biuf":
        raise _input_error(f"{field} must contain integers", field)
    bounds = np.iinfo(dtype)
    if source.size and (source.min() < bounds.min or source.max() > bounds.max):
        raise _input_error(f"{field} contains values outside {dtype} range", field)
    return np.array(source, dtype=dtype, order="C", copy=True)


def _input_error(message: str, field: str) -> _InputValidationError:
    return _InputValidationError(message, ("input", field))


__all__ = ["StructureBatch", "coerce_batch"]
