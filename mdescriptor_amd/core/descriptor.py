"""Lifecycle and the single ``compute`` boundary of a descriptor.

Same contract as ``src/mdescriptor/core/descriptor.py:29-147``: input is
coerced and validated before any device work, cancellation is checked before
and after, ``close()`` is final, and an active descriptor cannot be pickled.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from copy import deepcopy
from typing import Any, ClassVar

from .errors import (
    CancelledError,
    ClosedDescriptorError,
    DescriptorInputError,
    MDescriptorError,
    _InputValidationError,
)
from .input import coerce_batch
from .options import CONFIGURATION_SCHEMA_VERSION
from .result import DescriptorResult


class DescriptorConfiguration:
    """Versioned JSON-safe construction snapshot (options.py:61-128)."""

    __slots__ = ("schema_version", "descriptor", "parameters")

    def __init__(self, schema_version: int, descriptor: str, parameters: dict[str, Any]) -> None:
        self.schema_version = int(schema_version)
        self.descriptor = str(descriptor)
        self.parameters = deepcopy(parameters)

    def to_dict(self) -> dict[str, Any]:
        return {"schema_version": self.schema_version, "descriptor": self.descriptor,
                "parameters": deepcopy(self.parameters)}


class Descriptor(ABC):
    name: ClassVar[str]

    def __init__(self) -> None:
        self._closed = False
        self._configuration = DescriptorConfiguration(CONFIGURATION_SCHEMA_VERSION, self.name, {})
        self._metadata_snapshot: dict[str, Any] = {}

    @property
    def closed(self) -> bool:
        return self._closed

    @property
    def feature_count(self) -> int | None:
        return None

    @property
    def configuration(self) -> DescriptorConfiguration:
        return self._configuration

    @property
    def metadata(self) -> dict[str, Any]:
        return deepcopy(self._metadata_snapshot)

    def _set_configuration(self, schema_version: int, parameters: dict[str, Any]) -> None:
        self._configuration = DescriptorConfiguration(schema_version, self.name, parameters)

    def compute(self, value: Any, *, control: Any = None) -> DescriptorResult:
        """Compute one batch (descriptor.py:75-112)."""

        self._ensure_open()
        if _is_cancelled(control):
            raise CancelledError("descriptor computation was cancelled")
        try:
            batch = coerce_batch(value)
            self._validate_batch(batch)
        except DescriptorInputError:
            raise
        except (TypeError, ValueError) as exc:
            path = list(exc.path) if isinstance(exc, _InputValidationError) else ["input"]
            raise DescriptorInputError(str(exc), path=path) from exc
        result = self._compute_batch(batch, control=control)
        if _is_cancelled(control):
            raise CancelledError("descriptor computation was cancelled")
        if not isinstance(result, DescriptorResult):
            raise MDescriptorError(f"{self.name} returned {type(result).__name__}, expected DescriptorResult")
        return result

    @abstractmethod
    def _compute_batch(self, batch: Any, *, control: Any = None) -> DescriptorResult:
        raise NotImplementedError

    def _validate_batch(self, batch: Any) -> None:
        del batch

    def close(self) -> None:
        self._closed = True

    def __enter__(self) -> Descriptor:
        self._ensure_open()
        return self

    def __exit__(self, exc_type: Any, exc_value: Any, traceback: Any) -> None:
        self.close()

    def __getstate__(self) -> Any:
        raise TypeError("active descriptors are not pickleable; store a JSON configuration and rebuild")

    def _ensure_open(self) -> None:
        if self._closed:
            raise ClosedDescriptorError(f"descriptor {self.name!r} is closed")


def _is_cancelled(control: Any) -> bool:
    if control is None:
        return False
    checker = getattr(control, "cancelled", None)
    if checker is None:
        return False
    return bool(checker() if callable(checker) else checker)


__all__ = ["Descriptor", "DescriptorConfiguration"]
