from .neighbor import NeighborSampler  # noqa: F401

__all__ = ["NeighborSampler"]
