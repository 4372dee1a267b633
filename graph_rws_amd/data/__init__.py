from .bcsr import BCSRGraph  # noqa: F401
from .layout import aligned_rows  # noqa: F401
from .loader import WindowWiseDataLoader  # noqa: F401

__all__ = ["BCSRGraph", "WindowWiseDataLoader", "aligned_rows"]
