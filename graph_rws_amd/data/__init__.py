from .bcsr import BCSRGraph  # noqa: F401

__all__ = ["BCSRGraph"]
