"""MDescriptor's SOAP descriptor on AMD Instinct MI355X (gfx950).

The public names match the reference package (``src/mdescriptor/__init__.py``)
for the SOAP path: build a :class:`StructureBatch`, construct
``SOAP(species=..., r_cut=..., execution=ExecutionOptions(device="hip"))`` and
call ``compute``.  ``NeighborList`` gives the same device graph as a
pair-level result.  All numerical work runs in the HIP library
``mdescriptor_amd/_lib/libmdx_hip.so`` (C-ABI declared in
``include/mdx_hip.h``); there is no CPU execution path.
"""

from __future__ import annotations

from .core.control import ComputeControl
from .core.errors import (
    CancelledError,
    ClosedDescriptorError,
    DescriptorConfigError,
    DescriptorInputError,
    MDescriptorError,
    UnsupportedPeriodicityError,
)
from .core.input import StructureBatch
from .core.options import ExecutionOptions, OutputOptions
from .core.result import DescriptorLevel, DescriptorResult
from .descriptors.neighbor_list import NeighborList
from .descriptors.soap import SOAP

__version__ = "0.1.0"

__all__ = [
    "CancelledError",
    "ClosedDescriptorError",
    "ComputeControl",
    "DescriptorConfigError",
    "DescriptorInputError",
    "DescriptorLevel",
    "DescriptorResult",
    "ExecutionOptions",
    "MDescriptorError",
    "NeighborList",
    "OutputOptions",
    "SOAP",
    "StructureBatch",
    "UnsupportedPeriodicityError",
]
