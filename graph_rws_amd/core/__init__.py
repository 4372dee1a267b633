"""MI355X-native replacement of the reference's `core` package
(core/__init__.py:3-46).  Same exported names; every op runs the gfx950
kernels of libgrws.so through its C ABI (include/grws.h).  Unlike the
reference, a missing library is an error, not a silent `None`.
"""
from ._lib import load as _load  # noqa: F401
from .ops import (  # noqa: F401
    PackedTiles,
    pack_tiles,
    SpmmPlan,
    build_spmm_plan,
    csr_to_bcsr_cpu,
    default_slabs,
    SamplingTimingResult,
    reindex_bcsr,
    relabel,
    sample_all_layers,
    window_seeds,
    sample_hop,
    spmm,
    spmm_tc,
    spmm_transpose,
)


class SamplingConfig:
    """Lightweight config container for samplers (core/__init__.py:39-44)."""

    def __init__(self):
        self.sample_num = 128
        self.warps_per_block = 8
        self.large_window_threshold = 4096


__all__ = [
    "spmm_tc",
    "spmm_transpose",
    "reindex_bcsr",
    "csr_to_bcsr_cpu",
    "SamplingConfig",
    "spmm",
    "build_spmm_plan",
    "SpmmPlan",
    "PackedTiles",
    "pack_tiles",
    "sample_hop",
    "relabel",
    "sample_all_layers",
    "SamplingTimingResult",
    "window_seeds",
]
