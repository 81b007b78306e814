"""Errors of the public descriptor contract.

Same classes, codes and JSON shape as the reference
(``src/mdescriptor/core/errors.py:11-130``), so callers that catch or
serialise MDescriptor errors keep working.  The backend translation maps the
HIP plugin's exception families (see ``mdescriptor_amd._hip``).
"""

from __future__ import annotations

import math
from collections.abc import Mapping
from typing import Any


class MDescriptorError(Exception):
    """Root of every error the descriptor API raises.

    Carries a machine-readable ``code``, the location in the inputs that
    failed (``path``, optional) and JSON-safe ``details``; ``to_dict`` gives
    the serialised form."""

    default_code = "mdescriptor_error"

    def __init__(self, message: str = "", *, code: str | None = None, path: Any = None,
                 details: Mapping[str, Any] | None = None) -> None:
        self.message = str(message)
        self.code = str(code or self.default_code)
        self.path = _error_path(path)
        self.details = None if details is None else _json_details(details)
        Exception.__init__(self, self.message)

    def to_dict(self) -> dict[str, Any]:
        result: dict[str, Any] = {"code": self.code, "message": self.message}
        if self.path is not None:
            result["path"] = list(self.path)
        if self.details is not None:
            result["details"] = self.details
        return result


class _InputValidationError(ValueError):
    """ValueError raised while a field of the input is checked; ``path`` names
    that field so the public error can point at it."""

    def __init__(self, message: str, path: tuple[str | int, ...]) -> None:
        self.path = path
        super().__init__(message)


class DescriptorConfigError(MDescriptorError, ValueError):
    """Raised when the options of a descriptor (or what a backend declares it
    supports) are rejected."""

    default_code = "invalid_configuration"


class DescriptorInputError(MDescriptorError, ValueError):
    """Raised when a structure batch breaks the input rules of a descriptor."""

    default_code = "invalid_input"


class UnsupportedPeriodicityError(DescriptorInputError):
    """Raised for a batch whose periodicity the chosen descriptor cannot take."""

    default_code = "unsupported_periodicity"


class ClosedDescriptorError(MDescriptorError, RuntimeError):
    """Raised when a descriptor is used after ``close()``."""

    default_code = "closed_descriptor"


class CancelledError(MDescriptorError, RuntimeError):
    """Raised when a computation stops because its ``ComputeControl`` asked
    it to."""

    default_code = "cancelled"


def translate_backend_error(exc: Exception, *, unavailable_message: str, failure_message: str,
                            path: tuple[str, ...] | None = ("execution", "device"),
                            unavailable_details: bool = True) -> MDescriptorError:
    """Map one native-backend exception onto the public error schema
    (errors.py:83-117 of the reference)."""

    if isinstance(exc, MemoryError):
        return MDescriptorError("HIP backend ran out of memory", code="backend_out_of_memory", path=path)
    if isinstance(exc, (ImportError, OSError)):
        return MDescriptorError(
            unavailable_message,
            code="device_unavailable",
            path=path,
            details={"exception": type(exc).__name__} if unavailable_details else None,
        )
    return MDescriptorError(failure_message, code="backend_error", path=path,
                            details={"exception": type(exc).__name__})


def _error_path(value: Any) -> tuple[str | int, ...] | None:
    if value is None:
        return None
    if isinstance(value, (str, int)) and not isinstance(value, bool):
        return (value,)
    path = tuple(value)
    if any(not isinstance(item, (str, int)) or isinstance(item, bool) for item in path):
        raise TypeError("error path entries must be strings or integers")
    return path


def _json_details(value: Mapping[str, Any]) -> dict[str, Any]:
    def convert(item: Any) -> Any:
        if isinstance(item, Mapping):
            return {str(k): convert(v) for k, v in item.items()}
        if isinstance(item, (list, tuple)):
            return [convert(v) for v in item]
        if isinstance(item, float) and not math.isfinite(item):
            raise TypeError("error details cannot contain non-finite numbers")
        if item is None or isinstance(item, (str, int, float, bool)):
            return item
        if hasattr(item, "item"):
            return convert(item.item())
        raise TypeError(f"error detail is not JSON-safe: {type(item).__name__}")

    if not isinstance(value, Mapping):
        raise TypeError("error details must be a mapping")
    return convert(value)


__all__ = [
    "CancelledError",
    "ClosedDescriptorError",
    "DescriptorConfigError",
    "DescriptorInputError",
    "MDescriptorError",
    "UnsupportedPeriodicityError",
    "translate_backend_error",
]
