from .bcsr import BCSRGraph  # noqa: F401
from .bcsr_io import (bcsr_bin_paths, estimate_bcsr_bytes, load_bcsr_bins,  # noqa: F401
                      make_bcsr_stub, save_bcsr_bins)
from .layout import aligned_rows  # noqa: F401
from .loader import WindowWiseDataLoader  # noqa: F401

__all__ = ["BCSRGraph", "WindowWiseDataLoader", "aligned_rows", "bcsr_bin_paths", "estimate_bcsr_bytes",
           "load_bcsr_bins", "make_bcsr_stub", "save_bcsr_bins"]
