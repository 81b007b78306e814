"""Output and execution options of a descriptor.

Same two frozen option records as the reference
(``src/mdescriptor/core/options.py:24-58``).  The one difference is the device
vocabulary: this build adds ``"hip"`` (one AMD Instinct GPU through the
``libmdx_hip`` C-ABI).  ``"cpu"`` and ``"cuda"`` stay valid option values so
configurations written for the reference still parse, and a descriptor that
cannot run on them rejects them with the reference's ``unsupported_device``
error when it is constructed.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Literal

from .errors import DescriptorConfigError

CONFIGURATION_SCHEMA_VERSION = 1
DEVICES = ("cpu", "cuda", "hip")


@dataclass(frozen=True, slots=True)
class OutputOptions:
    """How a descriptor result is represented (options.py:24-36)."""

    dtype: Literal["float32", "float64"] = "float64"
    sparse: bool = False

    def __post_init__(self) -> None:
        if self.dtype not in {"float32", "float64"}:
            raise DescriptorConfigError("output dtype must be 'float32' or 'float64'")
        if not isinstance(self.sparse, bool):
            raise DescriptorConfigError("output sparse must be a boolean")

    def to_dict(self) -> dict[str, Any]:
        return {"dtype": self.dtype, "sparse": self.sparse}


@dataclass(frozen=True, slots=True)
class ExecutionOptions:
    """Where and how a descriptor is evaluated (options.py:39-58)."""

    device: str = "hip"
    num_threads: int | None = None

    def __post_init__(self) -> None:
        if not isinstance(self.device, str) or not self.device.strip():
            raise DescriptorConfigError("execution device cannot be empty")
        if self.device not in DEVICES:
            raise DescriptorConfigError(
                "execution device must be exactly 'cpu', 'cuda' or 'hip'",
                code="invalid_device",
                path=["device"],
                details={"supported": list(DEVICES)},
            )
        if isinstance(self.num_threads, bool):
            raise DescriptorConfigError("num_threads must be a positive integer or None")
        if self.num_threads is not None and (not isinstance(self.num_threads, int) or self.num_threads <= 0):
            raise DescriptorConfigError("num_threads must be positive or None")

    def to_dict(self) -> dict[str, Any]:
        return {"device": self.device, "num_threads": self.num_threads}


def coerce_options(value: Any, option_type: type[Any], name: str) -> Any:
    """Accept an option record or a mapping of its fields (adapter.py:47-55)."""

    if value is None:
        return option_type()
    if isinstance(value, option_type):
        return value
    if isinstance(value, dict):
        try:
            return option_type(**value)
        except TypeError as exc:
            raise DescriptorConfigError(f"invalid {name} options: {exc}", path=[name]) from exc
    raise DescriptorConfigError(f"{name} must be {option_type.__name__}", path=[name])


__all__ = ["CONFIGURATION_SCHEMA_VERSION", "DEVICES", "ExecutionOptions", "OutputOptions", "coerce_options"]
