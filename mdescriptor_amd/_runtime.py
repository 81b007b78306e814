"""Lazy factory for the HIP plugin (``src/mdescriptor/_runtime.py:78-125``).

``create_hip_backend`` is the counterpart of ``create_cuda_backend``: it
imports the plugin module on first use and asks it for a backend.  A missing
library or device surfaces as ``MDescriptorError(code="device_unavailable")``;
there is no CPU fallback.
"""

from __future__ import annotations

from collections.abc import Mapping
from typing import Any

from .core.errors import MDescriptorError, translate_backend_error


def create_hip_backend(name: str, options: Mapping[str, Any]) -> Any:
    try:
        from . import _hip

        return _hip.create_backend(name, options)
    except MDescriptorError:
        raise
    except (ImportError, OSError, MemoryError) as exc:
        raise translate_backend_error(
            exc,
            unavailable_message=f"HIP backend is unavailable for {name}: {exc}",
            failure_message=f"HIP backend failed for {name}",
        ) from exc


__all__ = ["create_hip_backend"]
