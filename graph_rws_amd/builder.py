"""On-device COO -> CSR -> BCSR construction and BCSR transpose.

Front end of the gfx950 builder kernels in csrc/bcsr_build.hip.
"""
from __future__ import annotations

from .core import _lib as L


def available() -> bool:
    """True when the loaded libgrws.so carries the device builder."""
    try:
        return hasattr(L.load(), "grws_build_csr_count")
    except ImportError:
        return False


def csr_to_bcsr_device(*args, **kwargs):
    raise NotImplementedError("device BCSR builder is not in this library build")


def transpose(graph):
    raise NotImplementedError("device BCSR transpose is not in this library build")
