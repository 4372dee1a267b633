from .neighbor import NeighborSampler  # noqa: F401
from .sampler import BCSRSampler  # noqa: F401

__all__ = ["BCSRSampler", "NeighborSampler"]
