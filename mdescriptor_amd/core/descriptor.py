"""Descriptor lifecycle: admission of a batch, cancellation, closing.

Every public entry that computes (``compute`` and the device-output
``SOAP.compute_into``) goes through the same two gates of the base class:

* ``_admit`` runs before any device work: the descriptor must be open, the
  control must not be cancelled, and the input is coerced to a
  :class:`StructureBatch` and checked by the family (``_validate_batch``);
  a ``TypeError``/``ValueError`` there surfaces as ``DescriptorInputError``
  with the validator's path (or ``["input"]``).
* ``_release`` runs after the device work: a cancellation requested in the
  meantime still wins over the result.

A closed descriptor stays closed and keeps its configuration and metadata;
a live one cannot be pickled.  Contract of
``src/mdescriptor/core/descriptor.py:29-147`` (messages and error classes).
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
from .input import StructureBatch, coerce_batch
from .options import CONFIGURATION_SCHEMA_VERSION
from .result import DescriptorResult

_CANCELLED = "descriptor computation was cancelled"
_NOT_PICKLEABLE = "active descriptors are not pickleable; store a JSON configuration and rebuild"


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


def cancel_requested(control: Any) -> bool:
    """True when ``control`` (anything with a ``cancelled`` attribute or
    method, or None) asks to stop."""

    flag = getattr(control, "cancelled", False) if control is not None else False
    if callable(flag):
        flag = flag()
    return bool(flag)


class Descriptor(ABC):
    """Base of the descriptor families; they implement ``_compute_batch``
    and may narrow the accepted input with ``_validate_batch``."""

    name: ClassVar[str]

    def __init__(self) -> None:
        self._closed = False
        self._configuration = DescriptorConfiguration(CONFIGURATION_SCHEMA_VERSION, self.name, {})
        self._metadata_snapshot: dict[str, Any] = {}

    # ------------------------------------------------------------- state
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

    # ------------------------------------------------------------- gates
    def _ensure_open(self) -> None:
        if self._closed:
            raise ClosedDescriptorError(f"descriptor {self.name!r} is closed")

    def _admit(self, value: Any, control: Any) -> StructureBatch:
        """The checked batch of ``value``; nothing has touched a device yet."""

        self._ensure_open()
        if cancel_requested(control):
            raise CancelledError(_CANCELLED)
        try:
            batch = coerce_batch(value)
            self._validate_batch(batch)
        except DescriptorInputError:
            raise
        except (TypeError, ValueError) as exc:
            where = list(exc.path) if isinstance(exc, _InputValidationError) else ["input"]
            raise DescriptorInputError(str(exc), path=where) from exc
        return batch

    @staticmethod
    def _release(control: Any) -> None:
        """Raise if the computation was cancelled while it ran."""

        if cancel_requested(control):
            raise CancelledError(_CANCELLED)

    # ------------------------------------------------------------- compute
    def compute(self, value: Any, *, control: Any = None) -> DescriptorResult:
        batch = self._admit(value, control)
        result = self._compute_batch(batch, control=control)
        self._release(control)
        if isinstance(result, DescriptorResult):
            return result
        raise MDescriptorError(f"{self.name} returned {type(result).__name__}, expected DescriptorResult")

    @abstractmethod
    def _compute_batch(self, batch: StructureBatch, *, control: Any = None) -> DescriptorResult:
        """One admitted batch through the family's backend."""

    def _validate_batch(self, batch: StructureBatch) -> None:
        """Family-specific input checks (none by default)."""

    # ------------------------------------------------------------- lifecycle
    def close(self) -> None:
        self._closed = True

    def __enter__(self) -> Descriptor:
        self._ensure_open()
        return self

    def __exit__(self, *exc_info: Any) -> None:
        self.close()

    def __getstate__(self) -> Any:
        raise TypeError(_NOT_PICKLEABLE)


__all__ = ["Descriptor", "DescriptorConfiguration", "cancel_requested"]
