"""Species declarations: the atomic numbers a descriptor is built for.

Public contract of ``src/mdescriptor/core/species.py:16-86`` (function names,
error classes, messages and the ``path`` of each error).  A declaration is a
non-empty sequence of unique positive atomic numbers; each entry may be any
value ``int()`` accepts, except booleans and floats with a fractional part.
"""

from __future__ import annotations

from collections.abc import Iterable
from typing import Any

import numpy as np

from .errors import DescriptorConfigError, DescriptorInputError

_NOT_A_SEQUENCE = "species must be a sequence of atomic numbers"
_NOT_INTEGER = "species must contain integer atomic numbers"
_NOT_FINITE = "species must contain finite integer atomic numbers"
_NOT_UNIQUE = "species must be a non-empty sequence of unique atomic numbers"
_NOT_POSITIVE = "species must contain positive atomic numbers"


def _config_error(message: str) -> DescriptorConfigError:
    return DescriptorConfigError(message, path=["species"])


def _atomic_number(entry: Any) -> int:
    """One declared entry as an int, or the declaration's error."""

    if isinstance(entry, (bool, np.bool_)):
        raise _config_error(_NOT_INTEGER)
    try:
        number = int(entry)
    except (TypeError, ValueError, OverflowError) as exc:
        raise _config_error(_NOT_INTEGER) from exc
    if isinstance(entry, (float, np.floating)):
        # int() truncates: a float entry must already be that integer
        if not np.isfinite(entry):
            raise _config_error(_NOT_FINITE)
        if float(entry) != number:
            raise _config_error(_NOT_INTEGER)
    return number


def normalize_species(species: Iterable[int] | None) -> tuple[int, ...] | None:
    """The declaration as a tuple of ints (None stays None)."""

    if species is None:
        return None
    try:
        entries = list(species)
    except TypeError as exc:
        raise _config_error(_NOT_A_SEQUENCE) from exc
    # every entry is checked before the set-level rules
    declared = tuple(_atomic_number(entry) for entry in entries)
    if len(set(declared)) != len(declared) or not declared:
        raise _config_error(_NOT_UNIQUE)
    if min(declared) <= 0:
        raise _config_error(_NOT_POSITIVE)
    return declared


def require_species(species: Iterable[int] | None, *, descriptor: str) -> tuple[int, ...]:
    """The declaration, which this descriptor cannot be built without."""

    declared = normalize_species(species)
    if declared is not None:
        return declared
    raise DescriptorConfigError(f"{descriptor} requires an explicit species declaration at construction",
                                path=["species"])


def validate_batch_species(batch: Any, species: Iterable[int], *, descriptor: str) -> tuple[int, ...]:
    """The declaration, after checking that every atom of the batch is one
    of the declared elements."""

    declared = require_species(species, descriptor=descriptor)
    present = np.unique(np.asarray(batch.numbers))
    undeclared = present[~np.isin(present, np.asarray(declared))]
    if undeclared.size:
        raise DescriptorInputError(
            f"{descriptor} input contains species outside its declaration: {[int(z) for z in undeclared]}",
            path=["input", "numbers"],
        )
    return declared


__all__ = ["normalize_species", "require_species", "validate_batch_species"]
