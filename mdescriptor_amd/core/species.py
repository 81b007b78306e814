"""Species declarations (``src/mdescriptor/core/species.py:16-86``)."""

from __future__ import annotations

from collections.abc import Iterable
from typing import Any

import numpy as np

from .errors import DescriptorConfigError, DescriptorInputError


def normalize_species(species: Iterable[int] | None) -> tuple[int, ...] | None:
    """Validate and freeze an optional atomic-number declaration (species.py:16-58)."""

    if species is None:
        return None
    try:
        raw = tuple(species)
    except TypeError as exc:
        raise DescriptorConfigError("species must be a sequence of atomic numbers", path=["species"]) from exc
    if any(isinstance(value, (bool, np.bool_)) for value in raw):
        raise DescriptorConfigError("species must contain integer atomic numbers", path=["species"])
    try:
        values = tuple(int(value) for value in raw)
    except (TypeError, ValueError, OverflowError) as exc:
        raise DescriptorConfigError("species must contain integer atomic numbers", path=["species"]) from exc
    for original, value in zip(raw, values):
        if isinstance(original, (float, np.floating)):
            if not np.isfinite(original):
                raise DescriptorConfigError("species must contain finite integer atomic numbers", path=["species"])
            if float(original) != value:
                raise DescriptorConfigError("species must contain integer atomic numbers", path=["species"])
    if not values or len(set(values)) != len(values):
        raise DescriptorConfigError("species must be a non-empty sequence of unique atomic numbers", path=["species"])
    if any(value <= 0 for value in values):
        raise DescriptorConfigError("species must contain positive atomic numbers", path=["species"])
    return values


def require_species(species: Iterable[int] | None, *, descriptor: str) -> tuple[int, ...]:
    normalized = normalize_species(species)
    if normalized is None:
        raise DescriptorConfigError(
            f"{descriptor} requires an explicit species declaration at construction", path=["species"]
        )
    return normalized


def validate_batch_species(batch: Any, species: Iterable[int], *, descriptor: str) -> tuple[int, ...]:
    """Reject a batch holding an element outside the declaration (species.py:72-86)."""

    normalized = require_species(species, descriptor=descriptor)
    missing = set(int(v) for v in np.unique(batch.numbers)) - set(normalized)
    if missing:
        raise DescriptorInputError(
            f"{descriptor} input contains species outside its declaration: {sorted(missing)}",
            path=["input", "numbers"],
        )
    return normalized


__all__ = ["normalize_species", "require_species", "validate_batch_species"]
