"""Descriptor families implemented on the HIP library: SOAP and NeighborList."""

from .neighbor_list import NeighborList
from .soap import SOAP

__all__ = ["NeighborList", "SOAP"]
