"""Descriptor families implemented on the HIP library: SOAP."""

from .soap import SOAP

__all__ = ["SOAP"]
