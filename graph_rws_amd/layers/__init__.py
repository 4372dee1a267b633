from .layer import BCSRSPMMFunction, BCSRGraphConv  # noqa: F401
