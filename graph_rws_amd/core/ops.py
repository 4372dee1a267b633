"""Reference-named ops over libgrws.so.

Each function keeps the name, argument meaning and return shape of the
reference's pybind11 op it replaces (core/wrapper/bind.cpp:99-159) and runs
the hand-written gfx950 kernels through the C ABI.  Outputs and workspaces are
allocated here with torch's caching allocator; the library allocates nothing.
"""
from __future__ import annotations

import ctypes
import weakref
import os
from typing import Optional, Tuple

import torch

from . import _lib as L

# spmm_tc timing (the reference returns the kernel ms measured with a host
# sync per call, timer.h:22-52).  Off by default: ms is reported as 0.0 and
# no synchronisation happens.  Set to True to time each call with events.
TIMING = False
# SpMM over grouped tiles where a graph has them (False: packed or dense tiles)
GROUPED = True

# Graphs multiplied more than once read their values from packed tiles
# (BCSRGraph.packed_tiles); False keeps every SpMM on the dense tiles.
PACK_TILES = True


# ---------------------------------------------------------------------------
# SpMM plan
# ---------------------------------------------------------------------------
class SpmmPlan:
    """Device work schedule of one BCSR graph (see grws_spmm_plan in
    include/grws.h).  Built once per graph and reused by every SpMM call."""

    def __init__(self, items: torch.Tensor, split: torch.Tensor, counts, slabs: int):
        self.items = items
        self.split = split
        self.num_items, self.num_split, self.num_slots = (int(c) for c in counts)
        self.slabs_per_item = int(slabs)

    def view(self) -> L.SpmmPlanView:
        return L.SpmmPlanView(L.ptr(self.items), L.ptr(self.split), self.num_items,
                              self.num_split, self.num_slots, self.slabs_per_item, 0)


class spmm_tuning:
    """Context manager that sets SpMM dispatch overrides (grws_spmm_set_tuning;
    benchmarks and tests only) and restores the previous values on exit:
    ``with spmm_tuning(GRWS_SPMM_WAVES=2): ...``.  Process-wide: no other
    thread may be in an SpMM call meanwhile."""

    def __init__(self, **overrides: int):
        self.overrides = {k: int(v) for k, v in overrides.items()}
        self.saved = {}

    def __enter__(self):
        lib = L.load()
        for k, v in self.overrides.items():
            self.saved[k] = int(lib.grws_spmm_get_tuning(k.encode()))
            L.call("grws_spmm_set_tuning", k.encode(), v)
        return self

    def __exit__(self, *exc):
        for k, v in self.saved.items():
            L.call("grws_spmm_set_tuning", k.encode(), v)
        return False


def grouped_slab_pairs() -> bool:
    """Whether 4-window grouped products multiply slab pairs on the
    16x16x32 MFMA (the default) rather than single slabs (GRWS_GRP_K32=0)."""
    return int(L.load().grws_spmm_get_tuning(b"GRWS_GRP_K32")) != 0


def grouped_kernel(group_size: int) -> str:
    """The kernel a grouped product of `group_size` windows runs: slab pairs
    staged by direct loads into LDS (spmm_grp2d_kernel, the default), the
    same through registers (spmm_grp2_kernel, GRWS_GRP_DMA=0), or single
    slabs (spmm_grp_kernel: GRWS_GRP_K32=0, or groups of 2 or 8)."""
    if group_size != 4 or not grouped_slab_pairs():
        return "spmm_grp_kernel"
    return "spmm_grp2_kernel" if int(L.load().grws_spmm_get_tuning(b"GRWS_GRP_DMA")) == 0 else "spmm_grp2d_kernel"


def default_slabs(num_windows: int, num_tiles: int, tile_cols: int, n_cols: int) -> int:
    return int(L.load().grws_spmm_default_slabs(num_windows, num_tiles, tile_cols, n_cols))


# Longest items first within each XCD's eighth of the plan
# (grws_spmm_plan_order) when the plan splits windows: None = that rule,
# False = never, True = always.  Measured: c2 N=128 -5%, c4 N=112 -6.6%,
# N=256 -4.6%; c3 (community order, no split windows) +1% when forced
ORDER_ITEMS: Optional[bool] = None


def build_spmm_plan(window_offset: torch.Tensor, num_tiles: int, tile_cols: int,
                    slabs_per_item: int, order: Optional[bool] = None) -> SpmmPlan:
    """Builds the SpMM schedule on the device (one stream sync).  order:
    reorder the items longest first within each XCD's share
    (grws_spmm_plan_order); None follows ORDER_ITEMS (by default: when the
    plan splits windows, a power-law graph's hub windows)."""
    lib = L.load()
    dev = window_offset.device
    L.require_device("build_spmm_plan", dev, window_offset)
    if not window_offset.is_contiguous() or window_offset.dtype != torch.int64:
        raise RuntimeError("build_spmm_plan: window_offset must be a contiguous int64 tensor")
    W = window_offset.numel() - 1
    mi = ctypes.c_int64()
    ms = ctypes.c_int64()
    L.call("grws_spmm_plan_capacity", W, num_tiles, tile_cols, slabs_per_item,
           ctypes.byref(mi), ctypes.byref(ms))
    items = torch.empty(max(1, mi.value) * 4, dtype=torch.int32, device=dev)
    split = torch.empty(max(1, ms.value) * 3, dtype=torch.int32, device=dev)
    wsb = int(lib.grws_spmm_plan_workspace_bytes(W))
    ws = torch.empty(max(1, wsb), dtype=torch.uint8, device=dev)
    counts = (ctypes.c_int64 * 3)()
    L.call("grws_spmm_plan_build", L.ptr(window_offset), W, num_tiles, tile_cols, slabs_per_item,
           L.ptr(items), mi.value, L.ptr(split), ms.value, L.ptr(ws), wsb,
           ctypes.cast(counts, ctypes.POINTER(ctypes.c_int64)), L.stream_of(dev))
    if order is None:
        order = ORDER_ITEMS if ORDER_ITEMS is not None else counts[1] > 0
    if order and counts[0] > 1:
        owsb = int(lib.grws_spmm_plan_order_workspace_bytes(counts[0]))
        ows = torch.empty(max(1, owsb), dtype=torch.uint8, device=dev)
        L.call("grws_spmm_plan_order", L.ptr(items), counts[0], L.ptr(ows), owsb, L.stream_of(dev))
    return SpmmPlan(items, split, list(counts), slabs_per_item)


class TensorKey:
    """Cache key over tensors: valid while they are the same objects, not
    modified in place since (weak references, so a cache keeps nothing
    alive; an address reused by a new tensor does not match), plus plain
    values."""

    __slots__ = ("refs", "versions", "extra")

    def __init__(self, tensors, extra=()):
        self.refs = tuple(weakref.ref(t) for t in tensors)
        self.versions = tuple(t._version for t in tensors)
        self.extra = tuple(extra)

    def matches(self, tensors, extra=()) -> bool:
        return (len(tensors) == len(self.refs) and all(r() is t for r, t in zip(self.refs, tensors))
                and self.versions == tuple(t._version for t in tensors) and self.extra == tuple(extra))


def _tensor_cache(t: torch.Tensor) -> dict:
    """Per-tensor cache for raw-tensor calls (spmm_tc, spmm_transpose): a
    dict stored on the window_offset tensor object, so it lives exactly as
    long as the graph arrays do."""
    d = getattr(t, "_grws_cache", None)
    if d is None:
        d = {}
        t._grws_cache = d
    return d


def _cached_plan(window_offset: torch.Tensor, col_indices: torch.Tensor, tile_cols: int,
                 n_cols: int) -> SpmmPlan:
    num_tiles = col_indices.numel() // tile_cols
    W = window_offset.numel() - 1
    slabs = default_slabs(W, num_tiles, tile_cols, n_cols)
    key = (window_offset._version, col_indices.numel(), tile_cols, slabs)
    d = _tensor_cache(window_offset)
    hit = d.get("plan")
    if hit is None or hit[0] != key:
        hit = (key, build_spmm_plan(window_offset, num_tiles, tile_cols, slabs))
        d["plan"] = hit
    return hit[1]


def line_pitched_empty(rows: int, cols: int, dtype: torch.dtype, device, zero: bool = False) -> torch.Tensor:
    """A [rows, cols] view of a new buffer whose rows start on 128-byte
    lines (the row pitch rounded up to a multiple of 128 bytes).  Ragged
    widths (41 or 47 classes) made this way are gathered by the SpMM and
    widened to a multiple of 8 columns without a copy.  zero: the padding
    columns (and the values) start at zero; otherwise they are left as
    allocated."""
    esz = torch.empty(0, dtype=dtype).element_size()
    per = max(1, 128 // esz)
    pitch = (cols + per - 1) // per * per
    make = torch.zeros if zero else torch.empty
    return make((rows, pitch), dtype=dtype, device=device)[:, :cols]


def mm_line_pitched(a: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """a @ w (w cast to a's dtype) into a line-pitched output when the
    output width does not fill whole 128-byte lines (torch's GEMM writes
    the row-strided view directly); a plain matmul otherwise."""
    n = w.shape[1]
    if a.dim() != 2 or (n * a.element_size()) % 128 == 0:
        return torch.matmul(a, w)
    out = line_pitched_empty(a.shape[0], n, a.dtype, a.device)
    return torch.mm(a, w.to(a.dtype), out=out)


def pair_pitch(n: int, esz: int) -> int:
    """Row pitch (elements) of mm_pair_line_pitched's output: two products
    of width n, each padded to whole 128-byte lines."""
    per = max(1, 128 // esz)
    return 2 * ((n + per - 1) // per * per)


def fuse_self_pays(rows: int, n: int, esz: int) -> bool:
    """Whether to make X W_n and X W_s with one GEMM and add the self term in
    the SpMM's epilogue (measured on c3/c4): it saves the second pass over X
    and the separate add, but the SpMM then gathers rows of the paired
    output (twice the pitch) and reads the self term.  That pays for narrow
    outputs (the class layer: c4 3.19 -> 2.54 ms) and while the paired
    output stays within the 256 MB Infinity Cache (c3 hidden layers, even);
    a wide output past it lost (c4 hidden layer: 8.89 -> 9.05 ms)."""
    pitch_bytes = pair_pitch(n, esz) * esz
    return pitch_bytes <= 512 or rows * pitch_bytes <= (256 << 20)


def mm_pair_line_pitched(a: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor):
    """(a @ w1, a @ w2) from one GEMM over the weights side by side (cast to
    a's dtype): a [M, K], w1 and w2 [K, N].  Each product starts on a
    128-byte line of the shared output rows (N is padded with zero weight
    columns to whole lines), so both are line-pitched [M, N] views."""
    K, N = w1.shape
    npad = pair_pitch(N, a.element_size()) // 2
    if npad == N:
        w = torch.cat([w1, w2], 1).to(a.dtype)
    else:
        w = torch.zeros((K, 2 * npad), dtype=a.dtype, device=a.device)
        w[:, :N] = w1
        w[:, npad:npad + N] = w2
    ts = torch.matmul(a, w)
    return ts[:, :N], ts[:, npad:npad + N]


def _widen(t: torch.Tensor, vec: int) -> torch.Tensor:
    """t [R, C] as [R, C'] with C' = C rounded up to a multiple of vec,
    16-byte aligned rows: a strided view over the row padding t already
    has when its storage covers it (the extra columns then hold whatever
    the padding holds), otherwise a zero-padded copy whose rows start on
    128-byte lines (a 96-byte row at a 96-byte pitch straddles lines: the
    SpMM's gathers of such rows ran up to 26% slower).  Callers use the
    first C columns of any result that is column-separable."""
    R, C = t.shape
    Cp = -(-C // vec) * vec
    if C == Cp and t.stride(0) % vec == 0 and t.data_ptr() % 16 == 0:
        return t
    esz = t.element_size()
    if R > 0 and t.stride(1) == 1 and t.stride(0) >= Cp and t.stride(0) % vec == 0 \
            and t.data_ptr() % 16 == 0 \
            and (t.storage_offset() + (R - 1) * t.stride(0) + Cp) * esz <= t.untyped_storage().nbytes():
        return t.as_strided((R, Cp), (t.stride(0), 1))
    per = 128 // esz
    pitch = -(-Cp // per) * per
    out = torch.zeros((R, pitch), dtype=t.dtype, device=t.device)
    out[:, :C] = t
    return out[:, :Cp]


# ---------------------------------------------------------------------------
# packed tiles
# ---------------------------------------------------------------------------
class PackedTiles:
    """Compact copy of a 16x16-tile graph's values (grws_packed_tiles in
    include/grws.h): per tile 4 row groups of {mask_lo, mask_hi, start} and
    the nonzero values.  grws_spmm_packed reads it instead of the dense
    tiles and returns the same bits."""

    def __init__(self, header: torch.Tensor, values: torch.Tensor, num_values: int):
        self.header = header
        self.values = values
        self.num_values = int(num_values)

    def view(self) -> L.PackedTilesView:
        return L.PackedTilesView(L.ptr(self.header), L.ptr(self.values), self.num_values)

    def nbytes(self) -> int:
        return self.header.numel() * 4 + self.values.numel() * self.values.element_size()


def pack_tiles_supported(col_indices: torch.Tensor, values: torch.Tensor, tile_cols: int) -> bool:
    return (tile_cols == 16 and values.dtype in (torch.float16, torch.bfloat16) and values.is_cuda
            and values.is_contiguous() and values.data_ptr() % 8 == 0)


def pack_tiles(window_offset: torch.Tensor, col_indices: torch.Tensor, values: torch.Tensor,
               tile_cols: int) -> Optional[PackedTiles]:
    """Builds the packed tiles on the device (one stream sync), or returns
    None when the graph cannot be packed (tile shape, dtype, or more than
    2^30 - 16 nonzero values)."""
    if not pack_tiles_supported(col_indices, values, tile_cols):
        return None
    _check_graph(window_offset, col_indices, values, tile_cols)
    lib = L.load()
    dev = values.device
    L.require_device("pack_tiles", dev, window_offset, col_indices)
    W = window_offset.numel() - 1
    T = col_indices.numel() // tile_cols
    view = L.BcsrView(L.ptr(window_offset), L.ptr(col_indices), L.ptr(values), W, T, 16, tile_cols,
                      L.dtype_code(values.dtype), 0)
    wsb = int(lib.grws_pack_tiles_workspace_bytes(T))
    ws = torch.empty(max(1, wsb), dtype=torch.uint8, device=dev)
    nv = ctypes.c_int64()
    st = lib.grws_pack_tiles_count(ctypes.byref(view), L.ptr(ws), wsb, ctypes.byref(nv), L.stream_of(dev))
    if st == L.GRWS_E_CAPACITY:
        return None
    L.check("grws_pack_tiles_count", st)
    header = torch.empty(max(1, T * 12), dtype=torch.int32, device=dev)
    # 8 elements of padding the SpMM may read past the last value
    pvals = torch.zeros(nv.value + 8, dtype=values.dtype, device=dev)
    L.call("grws_pack_tiles_fill", ctypes.byref(view), L.ptr(header), L.ptr(pvals), nv.value, L.ptr(ws), wsb,
           L.stream_of(dev))
    return PackedTiles(header, pvals, nv.value)


class GroupedTiles:
    """A's tiles re-cut so that `group_size` consecutive windows share one
    sorted list of their columns, 16 per slab, with one packed 16x16
    sub-tile per window and slab (grws_grouped_tiles in include/grws.h).
    grws_spmm_grouped gathers every union column's X row once per group."""

    def __init__(self, group_offset, col_indices, header, values, num_groups, num_slabs, num_values,
                 max_group_slabs, num_cols, group_size, slot_ratio):
        self.group_offset = group_offset
        self.col_indices = col_indices
        self.header = header
        self.values = values
        self.num_groups = int(num_groups)
        self.num_slabs = int(num_slabs)
        self.num_values = int(num_values)
        self.max_group_slabs = int(max_group_slabs)
        self.num_cols = int(num_cols)
        self.group_size = int(group_size)
        # union column slots / the windows' own column slots
        self.slot_ratio = float(slot_ratio)

    def view(self) -> L.GroupedTilesView:
        return L.GroupedTilesView(L.ptr(self.group_offset), L.ptr(self.col_indices), L.ptr(self.header),
                                  L.ptr(self.values), self.num_groups, self.num_slabs, self.num_values,
                                  self.max_group_slabs, self.num_cols, self.group_size)

    def nbytes(self) -> int:
        return (self.group_offset.numel() * 8 + self.col_indices.numel() * 4 + self.header.numel() * 4
                + self.values.numel() * self.values.element_size())


# Build grouped tiles when the union of a group's columns is at most this
# share of its windows' own column slots (below it the saved gathers pay
# for the extra sub-tiles), and every group at most this many times the
# mean group's slabs (groups are not split across work-groups).
GROUP_MAX_RATIO = 0.8
GROUP_MAX_SKEW = 4.0
# windows per group: None picks by the product's width (group_size_for);
# an int fixes it
GROUP_SIZE = None
def group_size_for(n_cols: int) -> int:
    """Windows per group for products n_cols wide.  Four at every width
    measured on c3 (f16): N = 256 2.16 against 2.25 ms with two windows,
    N = 608 5.29 against 5.39 ms (320-column chunks, one window per wave);
    the saved intra-community gathers outweigh the added sub-tile headers.
    Eight ran slower at N = 608 (8.21 ms, two windows per wave).  Four-window
    groups multiply slab pairs on the 16x16x32 MFMA (N = 608 5.14 ms)."""
    if GROUP_SIZE:
        return int(GROUP_SIZE)
    return 4


# narrower products stay on the window-by-window kernel: a grouped chunk is
# at least 128 columns wide (measured on c3: N = 48 took twice as long)
GROUP_MIN_N = 192


def group_tiles(window_offset: torch.Tensor, col_indices: torch.Tensor, values: torch.Tensor, tile_cols: int,
                num_cols: int, group_size: Optional[int] = None, max_ratio: Optional[float] = None,
                max_skew: Optional[float] = None) -> Optional[GroupedTiles]:
    """Builds grouped tiles on the device (one stream sync), or returns None
    when they do not apply (dtype, shape) or would not pay: the union of the
    groups' columns above max_ratio of the windows' own column slots, or a
    group longer than max_skew times the mean."""
    if values.dtype not in (torch.float16, torch.bfloat16) or tile_cols not in (8, 16) or not values.is_cuda:
        return None
    _check_graph(window_offset, col_indices, values, tile_cols)
    group_size = (GROUP_SIZE or 4) if group_size is None else group_size
    max_ratio = GROUP_MAX_RATIO if max_ratio is None else max_ratio
    max_skew = GROUP_MAX_SKEW if max_skew is None else max_skew
    lib = L.load()
    dev = values.device
    L.require_device("group_tiles", dev, window_offset, col_indices)
    W = window_offset.numel() - 1
    T = col_indices.numel() // tile_cols
    if W == 0 or T == 0:
        return None
    view = L.BcsrView(L.ptr(window_offset), L.ptr(col_indices), L.ptr(values), W, T, 16, tile_cols,
                      L.dtype_code(values.dtype), 0)
    wsb = int(lib.grws_group_tiles_workspace_bytes(ctypes.byref(view), int(num_cols), int(group_size)))
    ws = torch.empty(max(1, wsb), dtype=torch.uint8, device=dev)
    ns, nv, mx = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    st = lib.grws_group_tiles_count(ctypes.byref(view), int(num_cols), int(group_size), L.ptr(ws), wsb,
                                    ctypes.byref(ns), ctypes.byref(nv), ctypes.byref(mx), L.stream_of(dev))
    if st == L.GRWS_E_CAPACITY:
        return None
    L.check("grws_group_tiles_count", st)
    S, NV, MX = ns.value, nv.value, mx.value
    Q = (W + group_size - 1) // group_size
    ratio = (16 * S) / max(1, T * tile_cols)
    if S == 0 or ratio > max_ratio or MX > max_skew * S / Q or NV > (1 << 30) - 16:
        return None
    goff = torch.empty(Q + 1, dtype=torch.int64, device=dev)
    gcols = torch.empty(S * 16, dtype=torch.int32, device=dev)
    header = torch.empty(S * group_size * 12, dtype=torch.int32, device=dev)
    gvals = torch.zeros(NV + 8, dtype=values.dtype, device=dev)  # 8 readable elements past the last
    L.call("grws_group_tiles_fill", ctypes.byref(view), int(num_cols), int(group_size), S, L.ptr(goff),
           L.ptr(gcols), L.ptr(header), L.ptr(gvals), NV, L.ptr(ws), wsb, L.stream_of(dev))
    return GroupedTiles(goff, gcols, header, gvals, Q, S, NV, MX, num_cols, group_size, ratio)


def grouped_supported(x: torch.Tensor, values: torch.Tensor) -> bool:
    """Whether grws_spmm_grouped takes x: 16-bit with the values' dtype,
    16-byte rows and a 16-byte aligned start."""
    return (x.dtype == values.dtype and x.dtype in (torch.float16, torch.bfloat16) and x.dim() == 2
            and x.stride(1) == 1 and x.shape[1] % 8 == 0 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0
            and x.shape[0] > 0)


# ---------------------------------------------------------------------------
# SpMM forward
# ---------------------------------------------------------------------------
def _check_graph(window_offset, col_indices, values, tile_cols):
    if not (window_offset.is_contiguous() and col_indices.is_contiguous() and values.is_contiguous()):
        raise RuntimeError("window_offset, original_col_indices and values_condensed must be contiguous")
    if window_offset.dtype != torch.int64:
        raise TypeError("window_offset must be int64")
    if col_indices.dtype != torch.int32:
        raise TypeError("original_col_indices must be int32")
    if tile_cols not in (8, 16):
        raise ValueError(f"tile_cols must be 8 or 16 (got {tile_cols})")
    if col_indices.numel() % tile_cols != 0:
        raise ValueError("original_col_indices length is not a multiple of tile_cols")
    if values.numel() != col_indices.numel() * 16:
        raise ValueError("values_condensed must hold 16*tile_cols values per tile")


def spmm(window_offset: torch.Tensor, col_indices: torch.Tensor, values: torch.Tensor,
         x: torch.Tensor, tile_cols: int, plan: Optional[SpmmPlan] = None,
         out: Optional[torch.Tensor] = None, packed: Optional[PackedTiles] = None,
         max_window_slabs: int = 0, residual: Optional[torch.Tensor] = None,
         grouped: Optional[GroupedTiles] = None) -> torch.Tensor:
    """Y[16W, N] = A X on the device (H1 kernel).  x: [x_rows, N] (row stride
    may exceed N); out dtype = x dtype.  packed: the graph's packed tiles
    (read instead of the dense values when x has the values' dtype).
    grouped: the graph's grouped tiles, used when x is a 16-bit matrix of
    the values' dtype with at most grouped.num_cols rows.
    max_window_slabs: an upper bound of every window's slabs when known
    (0 = unknown); lets a call without a plan use the buffer-load kernel.
    residual: R [r_rows, N] in x's dtype, added to the first r_rows rows of
    the product before rounding (Y = A X + R there)."""
    _check_graph(window_offset, col_indices, values, tile_cols)
    if residual is not None:
        if (residual.dim() != 2 or residual.shape[1] != x.shape[1] or residual.dtype != x.dtype
                or residual.stride(1) != 1 or residual.device != x.device):
            raise ValueError("residual must be [rows, N] with x's dtype and device and unit column stride")
    if not x.is_cuda:
        raise RuntimeError("input_B must be a CUDA tensor")
    if x.dim() != 2 or x.stride(1) != 1:
        raise RuntimeError("input_B must be 2-D with unit column stride (contiguous rows)")
    for t in (window_offset, col_indices, values):
        if t.device != x.device:
            raise RuntimeError("graph arrays and input_B must be on the same device")
    W = window_offset.numel() - 1
    N = x.shape[1]
    vec = 16 // x.element_size()
    if out is None and N % vec != 0 and W > 0:
        # The kernel's 16-byte gathers need whole vectors per row; a ragged
        # width (a 41-class output layer) would fall back to element loads.
        # Run on X widened to the next multiple and hand back the first N
        # columns of the result (columns are independent).
        x = _widen(x, vec)
        full = spmm(window_offset, col_indices, values, x, tile_cols, plan=plan, packed=packed,
                    max_window_slabs=max_window_slabs,
                    residual=None if residual is None else _widen(residual, vec), grouped=grouped)
        return full[:, :N]
    if out is None:
        out = torch.empty((W * 16, N), dtype=x.dtype, device=x.device)
    elif out.shape != (W * 16, N) or out.dtype != x.dtype or out.stride(1) != 1:
        raise ValueError("out must be [16W, N] with x's dtype and unit column stride")
    if W == 0 or N == 0:
        return out
    view = L.BcsrView(L.ptr(window_offset), L.ptr(col_indices), L.ptr(values), W,
                      col_indices.numel() // tile_cols, 16, tile_cols, L.dtype_code(values.dtype),
                      int(min(max(0, max_window_slabs), 2**31 - 1)))
    if (grouped is not None and GROUPED and grouped_supported(x, values) and x.shape[0] <= grouped.num_cols
            and N >= GROUP_MIN_N):
        gv = grouped.view()
        L.call("grws_spmm_grouped", ctypes.byref(view), ctypes.byref(gv), L.ptr(x), L.dtype_code(x.dtype),
               x.shape[0], x.stride(0), N, L.ptr(residual) if residual is not None else None,
               residual.stride(0) if residual is not None else 0,
               residual.shape[0] if residual is not None else 0, L.ptr(out), L.dtype_code(out.dtype),
               out.stride(0), L.stream_of(x.device))
        return out
    pv = None
    ws = None
    wsb = 0
    if plan is not None:
        pv = plan.view()
        wsb = int(L.load().grws_spmm_workspace_bytes(ctypes.byref(pv), N))
        if wsb:
            ws = torch.empty(wsb, dtype=torch.uint8, device=x.device)
    if residual is not None:
        pk = packed.view() if packed is not None and x.dtype == values.dtype else None
        L.call("grws_spmm_residual", ctypes.byref(view), ctypes.byref(pk) if pk is not None else None,
               ctypes.byref(pv) if pv is not None else None,
               L.ptr(x), L.dtype_code(x.dtype), x.shape[0], x.stride(0), N,
               L.ptr(residual), residual.stride(0), residual.shape[0], L.ptr(out),
               L.dtype_code(out.dtype), out.stride(0), L.ptr(ws), wsb, L.stream_of(x.device))
        return out
    if packed is not None and x.dtype == values.dtype:
        pk = packed.view()
        L.call("grws_spmm_packed", ctypes.byref(view), ctypes.byref(pk),
               ctypes.byref(pv) if pv is not None else None,
               L.ptr(x), L.dtype_code(x.dtype), x.shape[0], x.stride(0), N, L.ptr(out),
               L.dtype_code(out.dtype), out.stride(0), L.ptr(ws), wsb, L.stream_of(x.device))
        return out
    L.call("grws_spmm", ctypes.byref(view), ctypes.byref(pv) if pv is not None else None,
           L.ptr(x), L.dtype_code(x.dtype), x.shape[0], x.stride(0), N, L.ptr(out),
           L.dtype_code(out.dtype), out.stride(0), L.ptr(ws), wsb, L.stream_of(x.device))
    return out


def _cached_packed(window_offset: torch.Tensor, col_indices: torch.Tensor, values: torch.Tensor,
                   tile_cols: int) -> Optional[PackedTiles]:
    """Packed tiles for raw-tensor calls, with BCSRGraph.packed_tiles' rule:
    built on the second product of the same, unmodified arrays."""
    if not PACK_TILES or not pack_tiles_supported(col_indices, values, tile_cols):
        return None
    d = _tensor_cache(window_offset)
    ent = d.get("packed")
    if ent is None or not ent[0].matches((values, col_indices)):
        d["packed"] = (TensorKey((values, col_indices)), 1, None)
        return None
    key, calls, p = ent
    if p is None and calls == 1:
        p = pack_tiles(window_offset, col_indices, values, tile_cols) or False
        d["packed"] = (key, 2, p)
    return p or None


def spmm_tc(window_offset: torch.Tensor, original_col_indices: torch.Tensor,
            values_condensed: torch.Tensor, input_B: torch.Tensor, warps_per_block: int = 8,
            tile_cols: int = 8) -> Tuple[torch.Tensor, float]:
    """Drop-in for core_lib.spmm_tc (bind.cpp:124-130, spmm_wrapper.cu:33-95).

    Returns (C[16W, N], ms).  `warps_per_block` is accepted for API
    compatibility and ignored (the gfx950 kernel picks its own shape).
    `tile_cols` defaults to the reference's fixed 8 (config.h:17).  ms is 0.0
    unless ``graph_rws_amd.core.ops.TIMING`` is set.
    """
    plan = _cached_plan(window_offset, original_col_indices, tile_cols, input_B.shape[1])
    packed = None
    if input_B.dtype == values_condensed.dtype and input_B.is_cuda:
        packed = _cached_packed(window_offset, original_col_indices, values_condensed, tile_cols)
    if not TIMING:
        return spmm(window_offset, original_col_indices, values_condensed, input_B, tile_cols,
                    plan=plan, packed=packed), 0.0
    s = torch.cuda.current_stream(input_B.device)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(s)
    y = spmm(window_offset, original_col_indices, values_condensed, input_B, tile_cols, plan=plan,
             packed=packed)
    e1.record(s)
    e1.synchronize()
    return y, float(e0.elapsed_time(e1))


# ---------------------------------------------------------------------------
# SpMM transpose (backward)
# ---------------------------------------------------------------------------
def _cached_transpose(window_offset, col_indices, values, tile_cols: int, num_cols: int):
    extra = (int(num_cols), int(tile_cols))
    d = _tensor_cache(window_offset)
    hit = d.get("T")
    if hit is not None and hit[0].matches((window_offset, col_indices, values), extra):
        return hit[1]
    key = TensorKey((window_offset, col_indices, values), extra)
    from ..data.bcsr import BCSRGraph
    W = window_offset.numel() - 1
    g = BCSRGraph(num_nodes=16 * W, num_edges=0, tile_rows=16, tile_cols=tile_cols,
                  window_offset=window_offset, original_col_indices=col_indices,
                  values_condensed=values, device=window_offset.device, num_rows=16 * W,
                  num_cols=int(num_cols), values_dtype=values.dtype)
    AT = g.transpose()
    d["T"] = (key, AT)
    return AT


def spmm_transpose(window_offset: torch.Tensor, original_col_indices: torch.Tensor,
                   values_condensed: torch.Tensor, grad_out: torch.Tensor, num_cols: int,
                   tile_cols: int = 8) -> torch.Tensor:
    """Drop-in for core_lib.spmm_transpose (bind.cpp:133-140,
    spmm_wrapper.cu:109-152): grad_in[num_cols, D] = A^T grad_out.

    The reference scatters with fp32 atomics (spmm_tc.cuh:211-270); here the
    BCSR of A^T is built once on the device (cached per graph) and the
    forward kernel runs over it, so the result is deterministic, exact in
    int64 index math, and covers every D (no 1e-9 skip, no D > 1024 cut)."""
    _check_graph(window_offset, original_col_indices, values_condensed, tile_cols)
    if not grad_out.is_cuda:
        raise RuntimeError("grad_out must be a CUDA tensor")
    AT = _cached_transpose(window_offset, original_col_indices, values_condensed, tile_cols,
                           num_cols)
    Y = AT.spmm(grad_out.contiguous())
    n = int(num_cols)
    if Y.shape[0] >= n:
        return Y[:n]
    return torch.nn.functional.pad(Y, (0, 0, 0, n - Y.shape[0]))


# ---------------------------------------------------------------------------
# reindex (model.py:126-141 -> reindex.cuh:33-102)
# ---------------------------------------------------------------------------
def reindex_bcsr(col_indices: torch.Tensor, values_condensed: torch.Tensor,
                 active_windows: torch.Tensor, tile_rows: int = 16,
                 tile_cols: int = 8) -> torch.Tensor:
    """Drop-in for core_lib.reindex_bcsr (bind.cpp:153-159): returns the
    local column ids (new int32 tensor) and prunes `values_condensed` in
    place where a column's window is not among `active_windows` (sorted);
    its version counter is bumped as by any in-place op."""
    if not (col_indices.is_cuda and values_condensed.is_cuda and active_windows.is_cuda):
        raise RuntimeError("reindex_bcsr: all tensors must be CUDA tensors")
    if col_indices.dtype != torch.int32 or active_windows.dtype != torch.int32:
        raise TypeError("reindex_bcsr: col_indices and active_windows must be int32")
    if not (col_indices.is_contiguous() and values_condensed.is_contiguous()
            and active_windows.is_contiguous()):
        raise RuntimeError("reindex_bcsr: tensors must be contiguous")
    n = col_indices.numel()
    if n % tile_cols != 0 or values_condensed.numel() != n * tile_rows:
        raise ValueError("reindex_bcsr: values_condensed must hold tile_rows values per column slot")
    out = torch.empty_like(col_indices)
    L.call("grws_reindex_prune", L.ptr(col_indices), n, L.ptr(values_condensed),
           L.dtype_code(values_condensed.dtype), L.ptr(active_windows), active_windows.numel(),
           int(tile_rows), int(tile_cols), L.ptr(out), L.stream_of(col_indices.device))
    # the prune wrote through a raw pointer: bump the version so caches keyed
    # on it (packed tiles, the transpose) see the change
    torch.autograd.graph.increment_version(values_condensed)
    return out


# ---------------------------------------------------------------------------
# CSR -> BCSR on host cores
# ---------------------------------------------------------------------------
def host_threads() -> int:
    """Host worker threads: OMP_NUM_THREADS when set (the share of the
    machine this process may use), else the visible core count."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    return os.cpu_count() or 1


def csr_to_bcsr_cpu(num_rows: int, row_ptr: torch.Tensor, col_idx: torch.Tensor,
                    values: torch.Tensor, tile_rows: int, tile_cols: int,
                    num_threads: int = 0):
    """Drop-in for core_lib.csr_to_bcsr_cpu (bind.cpp:143-150,
    convert_wrapper.cpp:27-180).  CPU tensors in, CPU tensors out:
    (window_offset int64[W+1], original_col_indices int32, values_condensed f32)."""
    if row_ptr.device.type != "cpu":
        raise RuntimeError("row_ptr must be on CPU")
    if num_threads <= 0:
        num_threads = host_threads()
    rp = row_ptr.to(torch.int64).contiguous()
    ci = col_idx.to("cpu", torch.int32).contiguous()
    va = values.to("cpu", torch.float32).contiguous()
    num_rows = int(num_rows)
    if rp.numel() != num_rows + 1:
        raise ValueError("row_ptr must have num_rows + 1 entries")
    W = (num_rows + tile_rows - 1) // tile_rows
    win = torch.empty(W + 1, dtype=torch.int64)
    T = ctypes.c_int64()
    L.call("grws_csr_to_bcsr_host_count", num_rows, L.ptr(rp), L.ptr(ci), tile_rows, tile_cols,
           L.ptr(win), ctypes.byref(T), num_threads)
    cols = torch.empty(T.value * tile_cols, dtype=torch.int32)
    vals = torch.empty(T.value * tile_rows * tile_cols, dtype=torch.float32)
    L.call("grws_csr_to_bcsr_host_fill", num_rows, L.ptr(rp), L.ptr(ci), L.ptr(va), tile_rows,
           tile_cols, L.ptr(win), L.ptr(cols), L.ptr(vals), num_threads)
    return win, cols, vals


# ---------------------------------------------------------------------------
# node-wise fanout sampling + relabel (csrc/sample.hip)
# ---------------------------------------------------------------------------
def _csr_arrays(indptr: torch.Tensor, indices: torch.Tensor):
    if not (indptr.is_cuda and indices.is_cuda):
        raise RuntimeError("indptr and indices must be CUDA tensors")
    if indptr.dtype != torch.int64 or indices.dtype != torch.int32:
        raise TypeError("indptr must be int64 and indices int32")
    if not (indptr.is_contiguous() and indices.is_contiguous()):
        raise RuntimeError("indptr and indices must be contiguous")
    return indptr.numel() - 1, indices.numel()


def sample_hop(indptr: torch.Tensor, indices: torch.Tensor, frontier: torch.Tensor, fanout: int,
               seed: int = 42, with_values: bool = True):
    """One hop of node-wise sampling without replacement (Floyd over a
    Philox4x32-10 stream keyed by (seed, node, draw)).  Returns
    (edge_dst int32 [E] frontier positions, edge_src int64 [E] global ids,
    edge_val float32 [E] GCN weights or None), in frontier order then
    ascending CSR position.  One stream sync (the edge count)."""
    n, nnz = _csr_arrays(indptr, indices)
    dev = indptr.device
    fr = frontier.to(dev, torch.int64).contiguous()
    F = fr.numel()
    cap = max(1, F * int(fanout))
    dst = torch.empty(cap, dtype=torch.int32, device=dev)
    src = torch.empty(cap, dtype=torch.int64, device=dev)
    val = torch.empty(cap, dtype=torch.float32, device=dev) if with_values else None
    wsb = int(L.load().grws_sample_hop_workspace_bytes(F))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    E = ctypes.c_int64()
    L.call("grws_sample_hop", L.ptr(indptr), L.ptr(indices), n, nnz, L.ptr(fr), F, int(fanout),
           ctypes.c_uint64(int(seed) & 0xFFFFFFFFFFFFFFFF), L.ptr(dst), L.ptr(src), L.ptr(val), cap,
           L.ptr(ws), wsb, ctypes.byref(E), L.stream_of(dev))
    E = E.value
    return dst[:E], src[:E], (val[:E] if val is not None else None)


def relabel(frontier: torch.Tensor, edge_src: torch.Tensor, num_nodes: int):
    """Unique + relabel: frontier ids keep local ids [0, F); new source ids
    follow in ascending global id.  Returns (src_local int32 [E],
    next_frontier int64 [num_src]).  One stream sync."""
    dev = edge_src.device
    L.require_device("relabel", dev, edge_src)
    fr = frontier.to(dev, torch.int64).contiguous()
    es = edge_src.to(torch.int64).contiguous()
    F, E = fr.numel(), es.numel()
    src_local = torch.empty(max(E, 1), dtype=torch.int32, device=dev)
    nxt = torch.empty(max(F + E, 1), dtype=torch.int64, device=dev)
    wsb = int(L.load().grws_relabel_workspace_bytes(F, E))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    ns = ctypes.c_int64()
    L.call("grws_relabel", L.ptr(fr), F, L.ptr(es), E, int(num_nodes), L.ptr(src_local),
           L.ptr(nxt), max(F + E, 1), L.ptr(ws), wsb, ctypes.byref(ns), L.stream_of(dev))
    return src_local[:E], nxt[:ns.value]


# ---------------------------------------------------------------------------
# window top-K sampling (csrc/window_sample.hip): core_lib.sample_all_layers
# ---------------------------------------------------------------------------
class SamplingTimingResult:
    """Per-layer timing of sample_all_layers (bind.cpp:81-96): milliseconds
    of the column selection (phase 1, which here also records each column's
    source slot), the mapping (phase 2, folded into phase 1: 0.0), the
    recompression (phase 3) and the whole layer."""

    __slots__ = ("phase1_sampling_time", "phase2_mapping_time", "phase3_recompression_time",
                 "total_time")

    def __init__(self, p1: float = 0.0, p2: float = 0.0, p3: float = 0.0, total: float = 0.0):
        self.phase1_sampling_time = float(p1)
        self.phase2_mapping_time = float(p2)
        self.phase3_recompression_time = float(p3)
        self.total_time = float(total)

    def to_dict(self) -> dict:
        return {k: getattr(self, k) for k in self.__slots__}

    def __repr__(self) -> str:
        return ("SamplingTimingResult(phase1={:.3f}ms, phase2={:.3f}ms, phase3={:.3f}ms, "
                "total={:.3f}ms)".format(self.phase1_sampling_time, self.phase2_mapping_time,
                                         self.phase3_recompression_time, self.total_time))


def _window_seeds(ids: torch.Tensor, num_nodes: int, drop: bool):
    dev = ids.device
    L.require_device("window_seeds", dev, ids)
    ids = ids.to(torch.int32).contiguous()
    n = ids.numel()
    act = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    msk = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    wsb = int(L.load().grws_window_seeds_workspace_bytes(n))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    na = ctypes.c_int64()
    L.call("grws_window_seeds", L.ptr(ids), n, int(num_nodes), 16, 1 if drop else 0, L.ptr(act),
           L.ptr(msk), L.ptr(ws), wsb, ctypes.byref(na), L.stream_of(dev))
    return act[:na.value], msk[:na.value]


def window_seeds(seeds: torch.Tensor, num_nodes: int, drop_out_of_range: bool = False):
    """prepare_windows_and_masks (sampling_wrapper.cu:283-347): seed ids ->
    (sorted unique active windows int32, OR-ed row masks int32)."""
    return _window_seeds(seeds, num_nodes, drop_out_of_range)


def _hacs_view(dev, static_scores, window_part_ids, part_starts, part_ends, alpha, beta, delta,
               gamma_bonus, score_scale, use_hacs, locality_enabled, keep: list):
    if not use_hacs:
        return None
    def prep(t, dt):
        if t is None:
            return None
        t = torch.as_tensor(t).to(dev, dt).contiguous()
        keep.append(t)
        return t
    ss = prep(static_scores, torch.float32)
    if ss is None:
        raise RuntimeError("use_hacs needs static_scores")
    wp = ps = pe = None
    if locality_enabled:
        wp = prep(window_part_ids, torch.int32)
        ps = prep(part_starts, torch.int32)
        pe = prep(part_ends, torch.int32)
        if wp is None or ps is None or pe is None:
            raise RuntimeError("locality_enabled needs window_part_ids, part_starts and part_ends")
    return L.HacsView(L.ptr(ss), L.ptr(wp), L.ptr(ps), L.ptr(pe), ss.numel(),
                      0 if wp is None else wp.numel(), 0 if ps is None else min(ps.numel(), pe.numel()),
                      float(alpha), float(beta), float(delta), float(gamma_bonus), float(score_scale),
                      1, 1 if locality_enabled else 0)


# Key scratch lent to grws_window_topk for windows of more than 1,024 slots
# (their keys computed once, by many work-groups, instead of in the window's
# own work-group or once per selection pass); results do not depend on it
WINDOW_KEY_SCRATCH = 64 << 20


def sample_all_layers(window_offset: torch.Tensor, original_col_indices: torch.Tensor,
                      values_condensed: torch.Tensor, initial_seeds: torch.Tensor, fanouts,
                      num_global_nodes: int, static_scores: Optional[torch.Tensor] = None,
                      window_part_ids: Optional[torch.Tensor] = None,
                      part_starts: Optional[torch.Tensor] = None,
                      part_ends: Optional[torch.Tensor] = None, alpha: float = 1.0,
                      beta: float = 10.0, delta: float = 0.0, gamma_bonus: float = 0.0,
                      score_scale: float = 100.0, use_hacs: int = 0, locality_enabled: int = 0,
                      tile_rows: int = 16, tile_cols: int = 8, warps_per_block: int = 8,
                      with_timings: bool = True):
    """Drop-in for core_lib.sample_all_layers (bind.cpp:99-121 ->
    sampling_wrapper.cu:365-438).  Returns (layers, timings): per fanout, in
    the order given, [out_window_offset int64, out_col_indices int32 (global
    ids), out_values, active_windows int32, masks int32], and one
    SamplingTimingResult.  Output arrays are sized exactly (no -1 tail;
    views of buffers sized by the layers' bounds); values keep
    values_condensed's dtype.  warps_per_block is validated as the reference
    does (4 or 8) and has no effect on the result.  Every layer runs in one
    grws_window_sample_layers call: one host sync for the batch.
    with_timings=False (not in the reference) skips the phase timing events,
    which cost ~45 us of a c2 batch, and returns zero timings."""
    if tile_rows != 16 or tile_cols not in (8, 16):
        raise RuntimeError("sample_all_layers supports 16x8 tiles (the reference's) and 16x16")
    if warps_per_block not in (4, 8):
        raise RuntimeError(f"Unsupported warps_per_block: {warps_per_block}. Only 4 and 8 allowed.")
    _check_graph(window_offset, original_col_indices, values_condensed, tile_cols)
    if not window_offset.is_cuda:
        raise RuntimeError("window_offset must be a CUDA tensor")
    L.require_device("sample_all_layers", window_offset.device, original_col_indices, values_condensed)
    fanouts = [int(f) for f in fanouts]
    for f in fanouts:
        if not 1 <= f <= 256:
            raise RuntimeError("Fanout > 256 not supported (fanout must be in [1, 256])")
    if not fanouts:
        return [], []
    dev = window_offset.device
    W = window_offset.numel() - 1
    n_nodes = int(num_global_nodes) if int(num_global_nodes) > 0 else 16 * W
    keep: list = []
    hv = _hacs_view(dev, static_scores, window_part_ids, part_starts, part_ends, alpha, beta,
                    delta, gamma_bonus, score_scale, use_hacs, locality_enabled, keep)
    view = L.BcsrView(L.ptr(window_offset), L.ptr(original_col_indices), L.ptr(values_condensed),
                      W, original_col_indices.numel() // tile_cols, 16, tile_cols,
                      L.dtype_code(values_condensed.dtype), 0)
    seeds = initial_seeds.to(dev).to(torch.int32).contiguous()
    nl = len(fanouts)
    fan = (ctypes.c_int32 * nl)(*fanouts)
    max_a = (ctypes.c_int64 * nl)()
    max_t = (ctypes.c_int64 * nl)()
    L.call("grws_window_sample_layers_bounds", ctypes.byref(view), n_nodes, seeds.numel(), fan, nl, max_a, max_t)
    lib = L.load()
    bufs = []
    for i in range(nl):
        a, t = int(max_a[i]), int(max_t[i])
        bufs.append((torch.empty(a + 1, dtype=torch.int64, device=dev),
                     torch.empty(max(t * tile_cols, 1), dtype=torch.int32, device=dev),
                     torch.empty(max(t * 16 * tile_cols, 1), dtype=values_condensed.dtype, device=dev),
                     torch.empty(max(a, 1), dtype=torch.int32, device=dev),
                     torch.empty(max(a, 1), dtype=torch.int32, device=dev)))
    ptrs = [(ctypes.c_void_p * nl)(*[b[k].data_ptr() for b in bufs]) for k in range(5)]
    # plus key scratch for the big windows: at most the graph's slots, at
    # most WINDOW_KEY_SCRATCH bytes
    wsb = int(lib.grws_window_sample_layers_workspace_bytes(ctypes.byref(view), n_nodes, seeds.numel(), fan, nl))
    wsb += min(int(lib.grws_window_topk_key_scratch_bytes(ctypes.byref(view))), WINDOW_KEY_SCRATCH)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    counts = (ctypes.c_int64 * (2 * nl))()
    phase = (ctypes.c_float * (2 * nl))()
    L.call("grws_window_sample_layers", ctypes.byref(view), n_nodes, L.ptr(seeds), seeds.numel(), fan, nl,
           ctypes.byref(hv) if hv is not None else None, ptrs[0], ptrs[1], ptrs[2], ptrs[3], ptrs[4], counts,
           phase if with_timings else None, L.ptr(ws), wsb, L.stream_of(dev))
    layers, timings = [], []
    for i, (off, cols, vals, act, msk) in enumerate(bufs):
        A, T = int(counts[2 * i]), int(counts[2 * i + 1])
        layers.append([off[:A + 1], cols[:T * tile_cols], vals[:T * 16 * tile_cols], act[:A], msk[:A]])
        p1, p3 = float(phase[2 * i]), float(phase[2 * i + 1])
        timings.append(SamplingTimingResult(p1, 0.0, p3, p1 + p3))
    return layers, timings


class CapturedWindowSampler:
    """sample_all_layers replayed from a HIP graph: grws_window_sample_layers
    _enqueue captured once for a graph, its fanouts, its HACS settings and a
    seed-count capacity ``max_seeds``; any batch of at most max_seeds seeds
    replays it (the count is read on the device).  Per batch: the seeds
    staged by one copy, the replay, the layers' counts and error flags read
    back (the batch's one sync), then one copy launch hands out compact
    copies of the outputs, so a returned batch stays valid after later
    replays.  The layers are those sample_all_layers returns, bit for bit
    (no phase timings).  The graph arrays and score tables are held while
    the capture lives (it reads them through their addresses) and must not
    be modified meanwhile; one instance serves one stream at a time."""

    def __init__(self, window_offset: torch.Tensor, original_col_indices: torch.Tensor,
                 values_condensed: torch.Tensor, fanouts, num_global_nodes: int, max_seeds: int,
                 static_scores: Optional[torch.Tensor] = None, window_part_ids: Optional[torch.Tensor] = None,
                 part_starts: Optional[torch.Tensor] = None, part_ends: Optional[torch.Tensor] = None,
                 alpha: float = 1.0, beta: float = 10.0, delta: float = 0.0, gamma_bonus: float = 0.0,
                 score_scale: float = 100.0, use_hacs: int = 0, locality_enabled: int = 0, tile_cols: int = 8):
        if tile_cols not in (8, 16):
            raise RuntimeError("CapturedWindowSampler supports 16x8 tiles (the reference's) and 16x16")
        _check_graph(window_offset, original_col_indices, values_condensed, tile_cols)
        dev = window_offset.device
        L.require_device("CapturedWindowSampler", dev, original_col_indices, values_condensed)
        self.fanouts = [int(f) for f in fanouts]
        if not self.fanouts or any(not 1 <= f <= 256 for f in self.fanouts):
            raise RuntimeError("CapturedWindowSampler: one to 64 fanouts, each in [1, 256]")
        self.max_seeds = int(max_seeds)
        if self.max_seeds < 1:
            raise ValueError("CapturedWindowSampler: max_seeds must be at least 1")
        self.dev, self.tc = dev, int(tile_cols)
        self.arrays = (window_offset, original_col_indices, values_condensed)
        self.values_dtype = values_condensed.dtype
        W = window_offset.numel() - 1
        self.n_nodes = int(num_global_nodes) if int(num_global_nodes) > 0 else 16 * W
        self.keep: list = []
        self.hv = _hacs_view(dev, static_scores, window_part_ids, part_starts, part_ends, alpha, beta, delta,
                             gamma_bonus, score_scale, use_hacs, locality_enabled, self.keep)
        self.view = L.BcsrView(L.ptr(window_offset), L.ptr(original_col_indices), L.ptr(values_condensed), W,
                               original_col_indices.numel() // tile_cols, 16, tile_cols,
                               L.dtype_code(values_condensed.dtype), 0)
        nl = self.nl = len(self.fanouts)
        self.fan = (ctypes.c_int32 * nl)(*self.fanouts)
        max_a = (ctypes.c_int64 * nl)()
        max_t = (ctypes.c_int64 * nl)()
        L.call("grws_window_sample_layers_bounds", ctypes.byref(self.view), self.n_nodes, self.max_seeds, self.fan,
               nl, max_a, max_t)
        tc, lib = self.tc, L.load()
        self.bufs = []
        for i in range(nl):
            a, t = int(max_a[i]), int(max_t[i])
            self.bufs.append((torch.empty(a + 1, dtype=torch.int64, device=dev),
                              torch.empty(max(t * tc, 1), dtype=torch.int32, device=dev),
                              torch.empty(max(t * 16 * tc, 1), dtype=self.values_dtype, device=dev),
                              torch.empty(max(a, 1), dtype=torch.int32, device=dev),
                              torch.empty(max(a, 1), dtype=torch.int32, device=dev)))
        self.ptrs = [(ctypes.c_void_p * nl)(*[b[k].data_ptr() for b in self.bufs]) for k in range(5)]
        wsb = int(lib.grws_window_sample_layers_workspace_bytes(ctypes.byref(self.view), self.n_nodes,
                                                                self.max_seeds, self.fan, nl))
        wsb += min(int(lib.grws_window_topk_key_scratch_bytes(ctypes.byref(self.view))), WINDOW_KEY_SCRATCH)
        self.wsb = wsb
        self.ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        self.seeds_buf = torch.empty(self.max_seeds, dtype=torch.int32, device=dev)
        self.cnt_in = torch.zeros(1, dtype=torch.int64, device=dev)
        self.out_dev = torch.zeros(2 * nl + 1, dtype=torch.int64, device=dev)
        self.out_host = torch.empty(2 * nl + 1, dtype=torch.int64, pin_memory=True)
        # this capture's own second stream: the windows of over 1,024 slots
        # run on it beside the others (forked and joined with events, which
        # the capture records as two branches)
        self.side = torch.cuda.Stream(dev)
        self.graph = None
        self.replays = 0

    def _enqueue(self, stream) -> None:
        L.call("grws_window_sample_layers_enqueue", ctypes.byref(self.view), self.n_nodes, L.ptr(self.seeds_buf),
               self.max_seeds, L.ptr(self.cnt_in), self.fan, self.nl,
               ctypes.byref(self.hv) if self.hv is not None else None, self.ptrs[0], self.ptrs[1], self.ptrs[2],
               self.ptrs[3], self.ptrs[4], L.ptr(self.ws), self.wsb, L.ptr(self.out_dev),
               ctypes.c_void_p(stream.cuda_stream), ctypes.c_void_p(self.side.cuda_stream))

    def run(self, seeds: torch.Tensor):
        """The layers of sample_all_layers for these seeds (global node ids,
        any integer dtype, on any device): per fanout, in the order given,
        [window_offset, col_indices, values, active_windows, masks]."""
        sd = seeds.reshape(-1)
        F0 = int(sd.numel())
        if F0 > self.max_seeds:
            raise ValueError(f"CapturedWindowSampler: {F0} seeds above the capacity {self.max_seeds}")
        stream = torch.cuda.current_stream(self.dev)
        if F0:
            self.seeds_buf[:F0].copy_(sd.to(self.dev, torch.int32), non_blocking=True)
        self.cnt_in.fill_(F0)
        if self.graph is None:
            self._enqueue(stream)  # this batch, and every kernel loaded before the capture
            cs = torch.cuda.Stream(self.dev)
            cs.wait_stream(stream)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(cs):
                g.capture_begin(capture_error_mode="thread_local")
                try:
                    self._enqueue(cs)
                finally:
                    g.capture_end()
            stream.wait_stream(cs)
            self.graph = g
        else:
            self.graph.replay()
            self.replays += 1
        self.out_host.copy_(self.out_dev, non_blocking=True)
        stream.synchronize()
        c = self.out_host.tolist()
        if c[2 * self.nl]:
            L.call("grws_window_sample_layers_status", int(c[2 * self.nl]))
        # compact copies, one buffer per element type, segments on 16 bytes
        tc = self.tc
        seg64, seg32, segv = [], [], []
        for i, (off, cols, vals, act, msk) in enumerate(self.bufs):
            A, T = int(c[2 * i]), int(c[2 * i + 1])
            seg64.append((off, A + 1))
            seg32 += [(cols, T * tc), (act, A), (msk, A)]
            segv.append((vals, T * 16 * tc))
        esz = torch.empty(0, dtype=self.values_dtype).element_size()
        src, dst, nbytes, views = [], [], [], []
        for segs, dtype, es in ((seg64, torch.int64, 8), (seg32, torch.int32, 4), (segv, self.values_dtype, esz)):
            per = 16 // es
            offs, o = [], 0
            for _, k in segs:
                offs.append(o)
                o += -(-k // per) * per
            buf = torch.empty(max(o, per), dtype=dtype, device=self.dev)
            vs = []
            for (t, k), o in zip(segs, offs):
                if k:
                    src.append(t.data_ptr())
                    dst.append(buf.data_ptr() + o * es)
                    nbytes.append(k * es)
                vs.append(buf[o:o + k])
            views.append(vs)
        if src:
            m = len(src)
            L.call("grws_copy_ranges", (ctypes.c_void_p * m)(*src), (ctypes.c_void_p * m)(*dst),
                   (ctypes.c_int64 * m)(*nbytes), m, ctypes.c_void_p(stream.cuda_stream))
        v64, v32, vv = (iter(v) for v in views)
        layers = []
        for _ in range(self.nl):
            off = next(v64)
            cols, act, msk = next(v32), next(v32), next(v32)
            layers.append([off, cols, next(vv), act, msk])
        return layers


def _sample_all_layers_per_layer(window_offset: torch.Tensor, original_col_indices: torch.Tensor,
                      values_condensed: torch.Tensor, initial_seeds: torch.Tensor, fanouts,
                      num_global_nodes: int, static_scores: Optional[torch.Tensor] = None,
                      window_part_ids: Optional[torch.Tensor] = None,
                      part_starts: Optional[torch.Tensor] = None,
                      part_ends: Optional[torch.Tensor] = None, alpha: float = 1.0,
                      beta: float = 10.0, delta: float = 0.0, gamma_bonus: float = 0.0,
                      score_scale: float = 100.0, use_hacs: int = 0, locality_enabled: int = 0,
                      tile_rows: int = 16, tile_cols: int = 8, warps_per_block: int = 8):
    """sample_all_layers through the per-layer entry points (grws_window_seeds,
    grws_window_topk, grws_window_recompress; two host syncs per layer):
    the same results as the one-call path, kept to check it."""
    if tile_rows != 16 or tile_cols not in (8, 16):
        raise RuntimeError("sample_all_layers supports 16x8 tiles (the reference's) and 16x16")
    if warps_per_block not in (4, 8):
        raise RuntimeError(f"Unsupported warps_per_block: {warps_per_block}. Only 4 and 8 allowed.")
    _check_graph(window_offset, original_col_indices, values_condensed, tile_cols)
    if not window_offset.is_cuda:
        raise RuntimeError("window_offset must be a CUDA tensor")
    L.require_device("sample_all_layers", window_offset.device, original_col_indices, values_condensed)
    dev = window_offset.device
    W = window_offset.numel() - 1
    n_nodes = int(num_global_nodes) if int(num_global_nodes) > 0 else 16 * W
    keep: list = []
    hv = _hacs_view(dev, static_scores, window_part_ids, part_starts, part_ends, alpha, beta,
                    delta, gamma_bonus, score_scale, use_hacs, locality_enabled, keep)
    view = L.BcsrView(L.ptr(window_offset), L.ptr(original_col_indices), L.ptr(values_condensed),
                      W, original_col_indices.numel() // tile_cols, 16, tile_cols,
                      L.dtype_code(values_condensed.dtype), 0)
    stream = torch.cuda.current_stream(dev)
    seeds = initial_seeds.to(dev)
    active, masks = _window_seeds(seeds, n_nodes, drop=False)
    layers, timings = [], []
    fanouts = [int(f) for f in fanouts]
    for i, f in enumerate(fanouts):
        S = int(L.load().grws_window_sample_num(f))
        if not 1 <= f <= 256:
            raise RuntimeError("Fanout > 256 not supported (fanout must be in [1, 256])")
        A = active.numel()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        ev[0].record(stream)
        scols = torch.empty(max(A * S, 1), dtype=torch.int32, device=dev)
        sslot = torch.empty(max(A * S, 1), dtype=torch.int32, device=dev)
        out_off = torch.empty(A + 1, dtype=torch.int64, device=dev)
        # plus key scratch for the big windows (more than 1,024 slots): at
        # most the graph's slots, at most WINDOW_KEY_SCRATCH bytes
        wsb = int(L.load().grws_window_topk_workspace_bytes(A)) + min(
            int(L.load().grws_window_topk_key_scratch_bytes(ctypes.byref(view))), WINDOW_KEY_SCRATCH)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        T = ctypes.c_int64()
        L.call("grws_window_topk", ctypes.byref(view), L.ptr(active), A, f,
               ctypes.byref(hv) if hv is not None else None, L.ptr(scols), L.ptr(sslot),
               L.ptr(out_off), L.ptr(ws), wsb, ctypes.byref(T), L.stream_of(dev))
        T = T.value
        ev[1].record(stream)
        out_cols = torch.empty(T * tile_cols, dtype=torch.int32, device=dev)
        out_vals = torch.empty(T * 16 * tile_cols, dtype=values_condensed.dtype, device=dev)
        L.call("grws_window_recompress", ctypes.byref(view), L.ptr(active), A, f, L.ptr(scols),
               L.ptr(sslot), L.ptr(out_off), T, L.ptr(out_cols), L.ptr(out_vals),
               L.stream_of(dev))
        ev[2].record(stream)
        layers.append([out_off, out_cols, out_vals, active, masks])
        if i + 1 < len(fanouts):
            active, masks = _window_seeds(out_cols, n_nodes, drop=True)
        ev[2].synchronize()
        p1 = ev[0].elapsed_time(ev[1])
        p3 = ev[1].elapsed_time(ev[2])
        timings.append(SamplingTimingResult(p1, 0.0, p3, p1 + p3))
    return layers, timings


class SampleState:
    """Per-graph scratch of the fused samplers: a node -> local id map (int32,
    all -1 between calls) and the state words of grws_sample_blocks (uint32,
    all 0 between calls): the new-source bitmap (its first ceil(n/32) words,
    which grws_sample_block and the repack take), per-1024-id counts and the
    batch counters.  Every call leaves both as it found them.  One state
    serves one stream at a time."""

    def __init__(self, num_nodes: int, device):
        self.num_nodes = int(num_nodes)
        self.node_map = torch.empty(max(1, self.num_nodes), dtype=torch.int32, device=device)
        words = int(L.load().grws_sample_blocks_state_words(self.num_nodes))
        self.bitmap = torch.empty(max(4, words), dtype=torch.int32, device=device)
        self.reset()

    def reset(self) -> None:
        """Back to all -1 / all 0 (on the current stream)."""
        L.call("grws_sample_blocks_state_init", L.ptr(self.node_map), L.ptr(self.bitmap), self.num_nodes,
               L.stream_of(self.node_map.device))


def sample_block(indptr: torch.Tensor, indices: torch.Tensor, frontier: torch.Tensor, fanout: int,
                 state: SampleState, seed: int = 42, tile_cols: int = 16,
                 values_dtype: torch.dtype = torch.float32):
    """One hop in one call: fanout sampling, relabel and the hop's BCSR block
    (rows = frontier positions, columns = local source ids).  Returns
    (window_offset int64 [W+1], col_indices int32, values, next_frontier
    int64 [num_src], num_edges).  One stream sync."""
    n, nnz = _csr_arrays(indptr, indices)
    dev = indptr.device
    L.require_device("sample_block", dev, indices, state.node_map, state.bitmap)
    fr = frontier.to(dev, torch.int64).contiguous()
    F = fr.numel()
    lib = L.load()
    ms, mt = ctypes.c_int64(), ctypes.c_int64()
    L.call("grws_sample_block_capacity", F, int(fanout), int(tile_cols), ctypes.byref(ms),
           ctypes.byref(mt))
    W = (F + 15) // 16
    nxt = torch.empty(max(1, ms.value), dtype=torch.int64, device=dev)
    win = torch.empty(W + 1, dtype=torch.int64, device=dev)
    cols = torch.empty(max(1, mt.value * tile_cols), dtype=torch.int32, device=dev)
    vals = torch.empty(max(1, mt.value * 16 * tile_cols), dtype=values_dtype, device=dev)
    wsb = int(lib.grws_sample_block_workspace_bytes(F, int(fanout), n))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    counts = (ctypes.c_int64 * 3)()
    L.call("grws_sample_block", L.ptr(indptr), L.ptr(indices), n, nnz, L.ptr(fr), F, int(fanout),
           ctypes.c_uint64(int(seed) & 0xFFFFFFFFFFFFFFFF), L.ptr(state.node_map), L.ptr(state.bitmap),
           int(tile_cols), L.dtype_code(values_dtype), L.ptr(nxt), ms.value, L.ptr(win), L.ptr(cols),
           L.ptr(vals), mt.value, L.ptr(ws), wsb, ctypes.cast(counts, ctypes.POINTER(ctypes.c_int64)),
           L.stream_of(dev))
    E, S, T = (int(c) for c in counts)
    return win, cols[:T * tile_cols], vals[:T * 16 * tile_cols], nxt[:S], E


def copy_and_fill(copies, fills, stream: Optional[torch.cuda.Stream] = None) -> bool:
    """Device copies and int64 fills in one launch each (grws_copy_ranges,
    grws_fill_ranges_i64) on `stream` (the current stream by default).
    copies: (dst, src) pairs of contiguous tensors of equal byte size, both
    16-byte aligned; fills: (dst int64 contiguous tensor, value); every
    tensor on one device.  Returns False, with nothing done, when an operand
    does not qualify (the caller then copies with torch)."""
    if not copies and not fills:
        return True
    dev = (copies[0][0] if copies else fills[0][0]).device
    if any(t.device != dev for pair in copies for t in pair) or any(d.device != dev for d, _ in fills):
        return False
    for d, s_ in copies:
        if (not (d.is_cuda and s_.is_cuda and d.is_contiguous() and s_.is_contiguous())
                or d.data_ptr() % 16 or s_.data_ptr() % 16
                or d.numel() * d.element_size() != s_.numel() * s_.element_size()):
            return False
    for d, _ in fills:
        if not (d.is_cuda and d.dtype == torch.int64 and d.is_contiguous()):
            return False
    sp = ctypes.c_void_p((stream or torch.cuda.current_stream(dev)).cuda_stream)
    cp = [(d, s_) for d, s_ in copies if d.numel()]
    if cp:
        m = len(cp)
        L.call("grws_copy_ranges", (ctypes.c_void_p * m)(*[s_.data_ptr() for _, s_ in cp]),
               (ctypes.c_void_p * m)(*[d.data_ptr() for d, _ in cp]),
               (ctypes.c_int64 * m)(*[d.numel() * d.element_size() for d, _ in cp]), m, sp)
    fl = [(d, v) for d, v in fills if d.numel()]
    if fl:
        m = len(fl)
        L.call("grws_fill_ranges_i64", (ctypes.c_void_p * m)(*[d.data_ptr() for d, _ in fl]),
               (ctypes.c_int64 * m)(*[d.numel() for d, _ in fl]), (ctypes.c_int64 * m)(*[int(v) for _, v in fl]),
               m, sp)
    return True


def gather_rows(src: torch.Tensor, index: torch.Tensor, out: Optional[torch.Tensor] = None,
                err: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``src.index_select(0, index)`` for a 2-D device tensor whose rows are
    contiguous (any row pitch), in one launch of grws_gather_rows: the
    mini-batch producer's input features (engine.py:132-141 gathers
    ``features[input_nodes]``).  ``index`` is int64 or int32 on the same
    device.  An index outside [0, src.shape[0]) yields a zero row and, when
    ``err`` (an int32 device tensor the caller cleared) is given, sets
    ``err[0]`` to 1; no host sync either way."""
    if src.dim() != 2 or not src.is_cuda:
        raise ValueError("gather_rows: src must be a 2-D device tensor")
    if src.shape[1] > 1 and src.stride(1) != 1:
        raise ValueError("gather_rows: the rows of src must be contiguous")
    idx = index
    if idx.device != src.device:
        raise ValueError("gather_rows: index must be on src's device")
    if idx.dtype not in (torch.int64, torch.int32):
        idx = idx.to(torch.int64)
    idx = idx.contiguous().view(-1)
    n = idx.numel()
    D = src.shape[1]
    if out is None:
        out = torch.empty(n, D, dtype=src.dtype, device=src.device)
    elif out.shape != (n, D) or out.dtype != src.dtype or out.device != src.device or \
            (D > 1 and out.stride(1) != 1):
        raise ValueError("gather_rows: out must be a [n, D] tensor of src's dtype with contiguous rows")
    esz = src.element_size()
    if n == 0 or D == 0:
        return out
    L.call("grws_gather_rows", L.ptr(src), src.shape[0], src.stride(0) * esz, L.ptr(idx),
           int(idx.dtype == torch.int64), n, D * esz, L.ptr(out), out.stride(0) * esz,
           L.ptr(err) if err is not None else None, L.stream_of(src.device))
    return out


_BLOCKS_SIZES: dict = {}


def _sample_blocks_sizes(F0: int, fanouts, tile_cols: int, n: int):
    """Capacities and workspace of a batch shape (host arithmetic, cached)."""
    key = (F0, tuple(fanouts), tile_cols, n)
    hit = _BLOCKS_SIZES.get(key)
    if hit is None:
        H = len(fanouts)
        fo = (ctypes.c_int32 * H)(*[int(k) for k in fanouts])
        ms = (ctypes.c_int64 * H)()
        mt = (ctypes.c_int64 * H)()
        L.call("grws_sample_blocks_capacity", F0, fo, H, int(tile_cols), n,
               ctypes.cast(ms, ctypes.POINTER(ctypes.c_int64)), ctypes.cast(mt, ctypes.POINTER(ctypes.c_int64)))
        wsb = int(L.load().grws_sample_blocks_workspace_bytes(F0, fo, H, int(tile_cols), n))
        fcap = [F0] + [int(ms[h]) for h in range(H - 1)]
        hit = (fo, [int(x) for x in ms], [int(x) for x in mt], fcap, wsb)
        if len(_BLOCKS_SIZES) > 64:
            _BLOCKS_SIZES.clear()
        _BLOCKS_SIZES[key] = hit
    return hit


_BLOCKS_T_SIZES: dict = {}


def _sample_blocks_t_sizes(F0: int, fanouts, tile_cols: int, n: int, thops):
    """Transposed-block capacities and the workspace of a batch shape."""
    key = (F0, tuple(fanouts), tile_cols, n, tuple(thops))
    hit = _BLOCKS_T_SIZES.get(key)
    if hit is None:
        H = len(fanouts)
        fo = (ctypes.c_int32 * H)(*[int(k) for k in fanouts])
        th = (ctypes.c_int32 * H)(*[1 if t else 0 for t in thops])
        mw = (ctypes.c_int64 * H)()
        mt = (ctypes.c_int64 * H)()
        L.call("grws_sample_blocks_transposed_capacity", F0, fo, H, int(tile_cols), n,
               ctypes.cast(mw, ctypes.POINTER(ctypes.c_int64)), ctypes.cast(mt, ctypes.POINTER(ctypes.c_int64)))
        wsb = int(L.load().grws_sample_blocks_transposed_workspace_bytes(F0, fo, H, int(tile_cols), n, th))
        hit = (th, [int(x) for x in mw], [int(x) for x in mt], wsb)
        if len(_BLOCKS_T_SIZES) > 64:
            _BLOCKS_T_SIZES.clear()
        _BLOCKS_T_SIZES[key] = hit
    return hit


def sample_blocks(indptr: torch.Tensor, indices: torch.Tensor, seeds: torch.Tensor, fanouts,
                  state: SampleState, seed: int = 42, tile_cols: int = 16,
                  values_dtype: torch.dtype = torch.float32, transposes=None):
    """Every hop of a mini-batch in one call (fanouts in hop order, hop 0 from
    the seeds): per hop (window_offset, col_indices, values, next_frontier,
    num_edges) as sample_block returns them.  One stream sync for the whole
    batch; outputs are views of buffers sized by the hops' capacities.

    transposes: per hop, whether to build the transpose of its block in the
    same call (grws_sample_blocks_transposed); each hop's tuple then has a
    sixth entry, (t_window_offset, t_col_indices, t_values, most tiles in
    one window) for a transposed hop and None for another."""
    n, nnz = _csr_arrays(indptr, indices)
    dev = indptr.device
    L.require_device("sample_blocks", dev, indices, state.node_map, state.bitmap)
    sd = seeds.to(dev, torch.int64).contiguous()
    F0 = sd.numel()
    H = len(fanouts)
    fo, ms, mt, fcap, wsb = _sample_blocks_sizes(F0, fanouts, int(tile_cols), n)
    thops = None
    if transposes is not None:
        if len(transposes) != H:
            raise ValueError("sample_blocks: one transposes flag per hop")
        thops = [bool(t) for t in transposes]
    any_t = bool(thops) and any(thops)
    tw = tt = [0] * H
    if any_t:
        th, tw, tt, wsb = _sample_blocks_t_sizes(F0, fanouts, int(tile_cols), n, thops)
    tw = [tw[h] if any_t and thops[h] else 0 for h in range(H)]
    tt = [tt[h] if any_t and thops[h] else 0 for h in range(H)]

    # one buffer per element type, carved per hop on 256-byte boundaries
    def layout(sizes, esz):
        offs, o = [], 0
        for k in sizes:
            offs.append(o)
            o += -(-max(1, k) * esz // 256) * 256 // esz
        return offs, o
    i64_sizes = ([ms[h] for h in range(H)] + [(fcap[h] + 15) // 16 + 1 for h in range(H)]
                 + [tw[h] + 1 for h in range(H)])
    i64_offs, i64_total = layout(i64_sizes, 8)
    c_offs, c_total = layout([mt[h] * tile_cols for h in range(H)] + [tt[h] * tile_cols for h in range(H)], 4)
    esz = torch.empty(0, dtype=values_dtype).element_size()
    v_offs, v_total = layout([mt[h] * 16 * tile_cols for h in range(H)]
                             + [tt[h] * 16 * tile_cols for h in range(H)], esz)
    b64 = torch.empty(i64_total, dtype=torch.int64, device=dev)
    bc = torch.empty(c_total, dtype=torch.int32, device=dev)
    bv = torch.empty(v_total, dtype=values_dtype, device=dev)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    nxt = [b64[i64_offs[h]:i64_offs[h] + max(1, ms[h])] for h in range(H)]
    win = [b64[i64_offs[H + h]:i64_offs[H + h] + i64_sizes[H + h]] for h in range(H)]
    cols = [bc[c_offs[h]:c_offs[h] + max(1, mt[h] * tile_cols)] for h in range(H)]
    vals = [bv[v_offs[h]:v_offs[h] + max(1, mt[h] * 16 * tile_cols)] for h in range(H)]
    twin = [b64[i64_offs[2 * H + h]:i64_offs[2 * H + h] + tw[h] + 1] for h in range(H)]
    tcols = [bc[c_offs[H + h]:c_offs[H + h] + max(1, tt[h] * tile_cols)] for h in range(H)]
    tvals = [bv[v_offs[H + h]:v_offs[H + h] + max(1, tt[h] * 16 * tile_cols)] for h in range(H)]

    def parr(ts):
        return (ctypes.c_void_p * H)(*[t.data_ptr() for t in ts])

    per = 5 if any_t else 3
    counts = (ctypes.c_int64 * (per * H))()
    common = (L.ptr(indptr), L.ptr(indices), n, nnz, L.ptr(sd), F0, fo, H,
              ctypes.c_uint64(int(seed) & 0xFFFFFFFFFFFFFFFF), L.ptr(state.node_map), L.ptr(state.bitmap),
              int(tile_cols), L.dtype_code(values_dtype), parr(nxt), parr(win), parr(cols), parr(vals))
    if any_t:
        L.call("grws_sample_blocks_transposed", *common, th, parr(twin), parr(tcols), parr(tvals), L.ptr(ws),
               wsb, ctypes.cast(counts, ctypes.POINTER(ctypes.c_int64)), L.stream_of(dev))
    else:
        L.call("grws_sample_blocks", *common, L.ptr(ws), wsb, ctypes.cast(counts, ctypes.POINTER(ctypes.c_int64)),
               L.stream_of(dev))
    out = []
    F = F0
    for h in range(H):
        E, S, T = int(counts[per * h]), int(counts[per * h + 1]), int(counts[per * h + 2])
        W = (F + 15) // 16
        hop = (win[h][:W + 1], cols[h][:T * tile_cols], vals[h][:T * 16 * tile_cols], nxt[h][:S], E)
        if thops is not None:
            t = None
            if thops[h]:
                TT, TM = int(counts[per * h + 3]), int(counts[per * h + 4])
                Wt = (S + 15) // 16
                t = (twin[h][:Wt + 1], tcols[h][:TT * tile_cols], tvals[h][:TT * 16 * tile_cols], TM)
            hop = hop + (t,)
        out.append(hop)
        F = S
    return out


class CapturedSampleBlocks:
    """sample_blocks replayed from a HIP graph: the batch's ~50 kernels
    (every hop's sampling, relabel, block and transpose builds) launched as
    one graph instead of one host launch each, which on a c5 batch cost more
    than the kernels themselves.

    One instance serves one batch shape: the CSR graph, the hop fanouts and
    transposes, the tile and dtype, the Philox seed, the SampleState and a
    seed-count capacity ``max_seeds``; any batch of at most max_seeds seeds
    replays it (grws_sample_blocks_enqueue reads the count on the device).
    The first call runs the enqueue eagerly and captures it; later calls copy
    the seeds into the static input, replay, read the counters back (the one
    sync of the batch, as in sample_blocks) and copy the outputs out of the
    static buffers into fresh compact tensors in one launch
    (grws_copy_ranges), so a returned batch stays valid after the next one.
    Returns what sample_blocks returns, bit for bit."""

    def __init__(self, indptr: torch.Tensor, indices: torch.Tensor, fanouts, state: "SampleState",
                 seed: int, tile_cols: int, values_dtype: torch.dtype, transposes, max_seeds: int):
        self.indptr, self.indices = indptr, indices
        n, nnz = _csr_arrays(indptr, indices)
        dev = indptr.device
        L.require_device("CapturedSampleBlocks", dev, state.node_map, state.bitmap)
        self.dev, self.n, self.nnz = dev, n, nnz
        self.H = H = len(fanouts)
        self.fanouts = [int(k) for k in fanouts]
        self.state = state
        self.seed = int(seed)
        self.tc = tc = int(tile_cols)
        self.values_dtype = values_dtype
        self.max_seeds = int(max_seeds)
        if self.max_seeds < 1:
            raise ValueError("CapturedSampleBlocks: max_seeds must be at least 1")
        fo, ms, mt, fcap, wsb = _sample_blocks_sizes(self.max_seeds, fanouts, tc, n)
        self.fo = fo
        thops = [bool(t) for t in transposes] if transposes is not None else [False] * H
        if len(thops) != H:
            raise ValueError("CapturedSampleBlocks: one transposes flag per hop")
        self.thops = thops
        tw, tt = [0] * H, [0] * H
        self.th = None
        if any(thops):
            self.th, tw, tt, wsb = _sample_blocks_t_sizes(self.max_seeds, fanouts, tc, n, thops)
            tw = [tw[h] if thops[h] else 0 for h in range(H)]
            tt = [tt[h] if thops[h] else 0 for h in range(H)]
        self.wsb = wsb
        self.esz = torch.empty(0, dtype=values_dtype).element_size()
        i64 = torch.int64
        # the seed count and the seeds the captured call reads; the count
        # arrives by a device copy from a table of [i, 0] pairs, in the same
        # launch as the seeds (16-byte aligned both)
        self.cnt_in = torch.zeros(2, dtype=i64, device=dev)
        self.seeds_buf = torch.empty(self.max_seeds, dtype=i64, device=dev)
        self.cnt_table = torch.stack([torch.arange(self.max_seeds + 1, dtype=i64),
                                      torch.zeros(self.max_seeds + 1, dtype=i64)], 1).contiguous().to(dev)
        self.pin = torch.empty(self.max_seeds, dtype=i64, pin_memory=True)
        self.nxt = [torch.empty(max(1, ms[h]), dtype=i64, device=dev) for h in range(H)]
        self.win = [torch.empty((fcap[h] + 15) // 16 + 1, dtype=i64, device=dev) for h in range(H)]
        self.cols = [torch.empty(max(1, mt[h] * tc), dtype=torch.int32, device=dev) for h in range(H)]
        self.vals = [torch.empty(max(1, mt[h] * 16 * tc), dtype=values_dtype, device=dev) for h in range(H)]
        self.twin = [torch.empty(tw[h] + 1, dtype=i64, device=dev) for h in range(H)]
        self.tcols = [torch.empty(max(1, tt[h] * tc), dtype=torch.int32, device=dev) for h in range(H)]
        self.tvals = [torch.empty(max(1, tt[h] * 16 * tc), dtype=values_dtype, device=dev) for h in range(H)]
        self.ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        self.cnt_dev = torch.zeros(5 * H + 2, dtype=i64, device=dev)
        self.cnt_host = torch.empty(5 * H + 2, dtype=i64, pin_memory=True)
        self.graph = None
        self.replays = 0

    def _parr(self, ts):
        return (ctypes.c_void_p * self.H)(*[t.data_ptr() for t in ts])

    def _enqueue(self, stream) -> None:
        L.call("grws_sample_blocks_enqueue", L.ptr(self.indptr), L.ptr(self.indices), self.n, self.nnz,
               L.ptr(self.seeds_buf), self.max_seeds, L.ptr(self.cnt_in), self.fo, self.H,
               ctypes.c_uint64(self.seed & 0xFFFFFFFFFFFFFFFF), L.ptr(self.state.node_map),
               L.ptr(self.state.bitmap), self.tc, L.dtype_code(self.values_dtype), self._parr(self.nxt),
               self._parr(self.win), self._parr(self.cols), self._parr(self.vals), self.th,
               self._parr(self.twin), self._parr(self.tcols), self._parr(self.tvals), L.ptr(self.ws), self.wsb,
               L.ptr(self.cnt_dev), ctypes.c_void_p(stream.cuda_stream))

    def run(self, seeds: torch.Tensor):
        F0 = int(seeds.numel())
        if F0 > self.max_seeds:
            raise ValueError(f"CapturedSampleBlocks: {F0} seeds above the capacity {self.max_seeds}")
        stream = torch.cuda.current_stream(self.dev)
        # stage the count and the seeds: contiguous int64 seeds on this
        # device, 16-byte aligned, and the count in one copy launch; other
        # device seeds by torch's copy (strides, dtype, device); host seeds
        # through the pinned buffer (free again: the previous call
        # synchronised after its copy)
        sd = seeds.reshape(-1)
        if (sd.is_cuda and sd.device == self.dev and sd.dtype == torch.int64 and sd.is_contiguous()
                and sd.data_ptr() % 16 == 0):
            srcs, dsts, nb = [self.cnt_table.data_ptr() + 16 * F0], [self.cnt_in.data_ptr()], [16]
            if F0:
                srcs.append(sd.data_ptr())
                dsts.append(self.seeds_buf.data_ptr())
                nb.append(8 * F0)
            m = len(srcs)
            L.call("grws_copy_ranges", (ctypes.c_void_p * m)(*srcs), (ctypes.c_void_p * m)(*dsts),
                   (ctypes.c_int64 * m)(*nb), m, ctypes.c_void_p(stream.cuda_stream))
        else:
            if sd.is_cuda:
                self.seeds_buf[:F0].copy_(sd.to(torch.int64))
            else:
                self.pin[:F0].copy_(sd.to(torch.int64))
                self.seeds_buf[:F0].copy_(self.pin[:F0], non_blocking=True)
            self.cnt_in.copy_(self.cnt_table[F0])
        if self.graph is None:
            self._enqueue(stream)  # this batch, and every kernel loaded before the capture
            cs = torch.cuda.Stream(self.dev)
            cs.wait_stream(stream)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(cs):
                g.capture_begin(capture_error_mode="thread_local")
                try:
                    self._enqueue(cs)
                finally:
                    g.capture_end()
            stream.wait_stream(cs)
            self.graph = g
        else:
            self.graph.replay()
            self.replays += 1
        self.cnt_host.copy_(self.cnt_dev, non_blocking=True)
        stream.synchronize()
        c = self.cnt_host.tolist()
        H = self.H
        if c[5 * H + 1]:
            L.call("grws_sample_blocks_error", int(c[5 * H + 1]))
        F = c[:H + 1]
        E = c[H + 1:2 * H + 1]
        T = c[2 * H + 1:3 * H + 1]
        TT = c[3 * H + 1:4 * H + 1]
        TM = c[4 * H + 1:5 * H + 1]
        tc, esz = self.tc, self.esz
        # compact outputs: one buffer per element type, segments on 16 bytes
        seg64, seg32, segv = [], [], []
        for h in range(H):
            seg64 += [(self.nxt[h], F[h + 1]), (self.win[h], (F[h] + 15) // 16 + 1)]
            seg32.append((self.cols[h], T[h] * tc))
            segv.append((self.vals[h], T[h] * 16 * tc))
            if self.thops[h]:
                seg64.append((self.twin[h], (F[h + 1] + 15) // 16 + 1))
                seg32.append((self.tcols[h], TT[h] * tc))
                segv.append((self.tvals[h], TT[h] * 16 * tc))

        def place(segs, dtype, esize):
            per = 16 // esize
            offs, o = [], 0
            for _, k in segs:
                offs.append(o)
                o += -(-k // per) * per
            buf = torch.empty(max(o, per), dtype=dtype, device=self.dev)
            return buf, offs
        b64, o64 = place(seg64, torch.int64, 8)
        b32, o32 = place(seg32, torch.int32, 4)
        bv, ov = place(segv, self.values_dtype, esz)
        src, dst, nbytes, views = [], [], [], []
        for segs, buf, offs, es in ((seg64, b64, o64, 8), (seg32, b32, o32, 4), (segv, bv, ov, esz)):
            vs = []
            for (t, k), o in zip(segs, offs):
                src.append(t.data_ptr())
                dst.append(buf.data_ptr() + o * es)
                nbytes.append(k * es)
                vs.append(buf[o:o + k])
            views.append(vs)
        m = len(src)
        L.call("grws_copy_ranges", (ctypes.c_void_p * m)(*src), (ctypes.c_void_p * m)(*dst),
               (ctypes.c_int64 * m)(*nbytes), m, ctypes.c_void_p(stream.cuda_stream))
        v64, v32, vv = (iter(v) for v in views)
        out = []
        for h in range(H):
            nxt, win = next(v64), next(v64)
            hop = (win, next(v32), next(vv), nxt, int(E[h]))
            t = None
            if self.thops[h]:
                t = (next(v64), next(v32), next(vv), int(TM[h]))
            out.append(hop + (t,) if any(self.thops) else hop)
        return out


# ---------------------------------------------------------------------------
# weight gradient A^T B (csrc/gemm_tn.hip)
# ---------------------------------------------------------------------------
def gemm_tn_supported(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Whether gemm_tn takes these operands: F16/BF16 2-D CUDA tensors with
    one dtype, equal row counts and unit column stride.  Widths or row
    strides that are not multiples of 8 (or rows not 16-byte aligned) are
    widened first (row padding reused when the storage covers it, a
    zero-padded copy otherwise)."""
    return (a.is_cuda and b.is_cuda and a.dim() == 2 and b.dim() == 2
            and a.dtype == b.dtype and a.dtype in (torch.float16, torch.bfloat16)
            and a.shape[0] == b.shape[0] and a.stride(1) == 1 and b.stride(1) == 1)


def gemm_tn(a: torch.Tensor, b: torch.Tensor, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """a^T @ b for a [K, M], b [K, N] (split over K, fp32 accumulation,
    deterministic); returns [M, N] in out_dtype (float32 or the inputs')."""
    if not gemm_tn_supported(a, b):
        raise ValueError("gemm_tn: unsupported operands (see gemm_tn_supported)")
    L.require_device("gemm_tn", a.device, b)
    K, M = a.shape
    N = b.shape[1]
    a2, b2 = _widen(a, 8), _widen(b, 8)
    M2, N2 = a2.shape[1], b2.shape[1]
    out = torch.empty((M2, N2), dtype=out_dtype, device=a.device)
    wsb = int(L.load().grws_gemm_tn_workspace_bytes(K, M2, N2))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=a.device)
    L.call("grws_gemm_tn", L.ptr(a2), a2.stride(0), L.ptr(b2), b2.stride(0), L.dtype_code(a.dtype), K,
           M2, N2, L.ptr(out), out.stride(0), L.dtype_code(out_dtype), L.ptr(ws), wsb,
           L.stream_of(a.device))
    if (M2, N2) != (M, N):
        out = out[:M, :N].contiguous()
    return out


# ---------------------------------------------------------------------------
# halo-aware subgraph repack (sampler/sampler.py:420-690)
# ---------------------------------------------------------------------------
class RepackResult:
    """Device outputs of one repack: the new window offsets, the input nodes
    (internal first, then the kept externals ascending), the halo and inner
    column / value arrays, the internal node count, and whether a halo value
    is NaN."""

    def __init__(self, window_offset, input_nodes, num_internal, halo_cols, halo_values, inner_cols,
                 inner_values, any_nan):
        self.window_offset = window_offset
        self.input_nodes = input_nodes
        self.num_internal = int(num_internal)
        self.halo_cols = halo_cols
        self.halo_values = halo_values
        self.inner_cols = inner_cols
        self.inner_values = inner_values
        self.any_nan = bool(any_nan)


def repack(window_offset: torch.Tensor, col_indices: torch.Tensor, values: torch.Tensor, tile_cols: int,
           num_nodes: int, window_ids: torch.Tensor, max_external_ratio: float, state: "SampleState",
           generator: Optional[torch.Generator] = None) -> RepackResult:
    """Repack of the selected windows on the device (csrc/repack.hip).

    window_ids: int64, strictly ascending, in [0, num_windows).  The external
    candidates are kept whole when they fit int(num_internal * ratio);
    otherwise a random subset of that size is kept, drawn as the reference
    draws it (one torch.randperm over the ascending candidates on the
    device, then sorted).  `state` is the graph's SampleState; it is left as
    found, also when a call fails."""
    _check_graph(window_offset, col_indices, values, tile_cols)
    dev = window_offset.device
    L.require_device("repack", dev, col_indices, values, window_ids, state.node_map, state.bitmap)
    if state.num_nodes < int(num_nodes):
        raise ValueError("repack: state is smaller than the graph")
    ids = window_ids.to(torch.int64).contiguous()
    n_sel = ids.numel()
    W = window_offset.numel() - 1
    view = L.BcsrView(L.ptr(window_offset), L.ptr(col_indices), L.ptr(values), W,
                      col_indices.numel() // tile_cols, 16, tile_cols, L.dtype_code(values.dtype), 0)
    lib = L.load()
    wsb = int(lib.grws_repack_workspace_bytes(n_sel, int(num_nodes)))
    ws = torch.empty(max(1, wsb), dtype=torch.uint8, device=dev)
    new_off = torch.empty(n_sel + 1, dtype=torch.int64, device=dev)
    counts = (ctypes.c_int64 * 3)()
    stream = L.stream_of(dev)
    L.call("grws_repack_prepare", ctypes.byref(view), int(num_nodes), L.ptr(ids), n_sel, L.ptr(state.bitmap),
           L.ptr(new_off), ctypes.cast(counts, ctypes.POINTER(ctypes.c_int64)), L.ptr(ws), wsb, stream)
    T, n_int, n_cand = (int(c) for c in counts)
    try:
        budget = int(n_int * max_external_ratio)
        kept = None
        n_kept = n_cand
        if n_cand > budget:
            ext = torch.empty(n_cand, dtype=torch.int64, device=dev)
            L.call("grws_repack_externals", L.ptr(state.bitmap), int(num_nodes), L.ptr(ext), L.ptr(ws), wsb, stream)
            perm = torch.randperm(n_cand, device=dev, generator=generator)
            kept = torch.sort(ext[perm[:budget]]).values.contiguous()
            n_kept = kept.numel()
        input_nodes = torch.empty(max(1, n_int + n_kept), dtype=torch.int64, device=dev)
        halo_cols = torch.empty(T * tile_cols, dtype=torch.int32, device=dev)
        inner_cols = torch.empty_like(halo_cols)
        halo_vals = torch.empty(T * 16 * tile_cols, dtype=values.dtype, device=dev)
        inner_vals = torch.empty_like(halo_vals)
        flags = (ctypes.c_int32 * 1)()
        L.call("grws_repack_finish", ctypes.byref(view), int(num_nodes), L.ptr(ids), n_sel, L.ptr(new_off), n_int,
               L.ptr(kept) if kept is not None else None, n_kept, L.ptr(state.node_map), L.ptr(state.bitmap),
               L.ptr(input_nodes), L.ptr(halo_cols), L.ptr(halo_vals), L.ptr(inner_cols), L.ptr(inner_vals),
               ctypes.cast(flags, ctypes.POINTER(ctypes.c_int32)), L.ptr(ws), wsb, stream)
    except BaseException:
        state.reset()
        raise
    return RepackResult(new_off, input_nodes[: n_int + n_kept], n_int, halo_cols, halo_vals, inner_cols,
                        inner_vals, flags[0])


# ---------------------------------------------------------------------------
# fused per-row epilogues (models/model.py:259-264, helper/engine.py:22-41)
# ---------------------------------------------------------------------------
def _rowwise_ok(t: torch.Tensor) -> bool:
    return (t.is_cuda and t.dim() == 2 and t.stride(1) == 1 and t.stride(0) % 4 == 0
            and t.data_ptr() % 8 == 0 and t.dtype in (torch.float32, torch.float16, torch.bfloat16))


def act_norm_dropout_supported(z: torch.Tensor) -> bool:
    """Whether the fused activation / LayerNorm / dropout kernel takes z."""
    return _rowwise_ok(z) and 4 <= z.shape[1] <= 1024 and z.shape[1] % 4 == 0


def _seed_dev(seed_dev: Optional[torch.Tensor], dev: torch.device):
    if seed_dev is None:
        return None
    if not (seed_dev.is_cuda and seed_dev.device == dev and seed_dev.dtype == torch.int64 and seed_dev.numel() >= 1):
        raise ValueError("seed_dev must be an int64 tensor with one element on the device of z")
    return L.ptr(seed_dev)


def act_norm_dropout_fwd(z: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float, p: float,
                         act: int, seed: int, out_dtype: torch.dtype, save_stats: bool,
                         seed_dev: Optional[torch.Tensor] = None):
    """out = dropout_p(LayerNorm(act(z))) (csrc/fused.hip); returns (out,
    mean, rstd) with mean/rstd None unless save_stats.  seed_dev: an int64
    device tensor whose first element the kernel reads in place of seed."""
    rows, dim = z.shape
    out = torch.empty((rows, dim), dtype=out_dtype, device=z.device)
    w = weight.detach().float().contiguous()
    b = bias.detach().float().contiguous()
    mean = rstd = None
    if save_stats:
        mean = torch.empty(max(1, rows), dtype=torch.float32, device=z.device)
        rstd = torch.empty_like(mean)
    L.call("grws_act_norm_dropout_fwd", L.ptr(z), L.dtype_code(z.dtype), z.stride(0), rows, dim, int(act),
           L.ptr(w), L.ptr(b), float(eps), float(p), int(seed) & ((1 << 64) - 1), _seed_dev(seed_dev, z.device),
           L.ptr(out), L.dtype_code(out_dtype), out.stride(0), L.ptr(mean), L.ptr(rstd), L.stream_of(z.device))
    return out, mean, rstd


def act_norm_dropout_bwd(dout: torch.Tensor, z: torch.Tensor, mean: torch.Tensor, rstd: torch.Tensor,
                         weight: torch.Tensor, p: float, act: int, seed: int,
                         seed_dev: Optional[torch.Tensor] = None):
    """(dz, dgamma, dbeta) of act_norm_dropout_fwd."""
    rows, dim = z.shape
    if not _rowwise_ok(dout):
        dout = dout.contiguous()
    dz = torch.empty_like(z, memory_format=torch.contiguous_format)
    dg = torch.empty(dim, dtype=torch.float32, device=z.device)
    db = torch.empty_like(dg)
    w = weight.detach().float().contiguous()
    wsb = int(L.load().grws_act_norm_dropout_bwd_workspace_bytes(rows, dim))
    ws = torch.empty(max(1, wsb), dtype=torch.uint8, device=z.device)
    L.call("grws_act_norm_dropout_bwd", L.ptr(dout), L.dtype_code(dout.dtype), dout.stride(0), L.ptr(z),
           L.dtype_code(z.dtype), z.stride(0), rows, dim, int(act), L.ptr(mean), L.ptr(rstd), L.ptr(w),
           float(p), int(seed) & ((1 << 64) - 1), _seed_dev(seed_dev, z.device), L.ptr(dz), dz.stride(0),
           L.ptr(dg), L.ptr(db), L.ptr(ws), wsb, L.stream_of(z.device))
    return dz, dg, db


def cross_entropy_fwd(logits: torch.Tensor, rows: Optional[torch.Tensor], labels: torch.Tensor):
    """(loss f32 scalar, counts int64 [3] = {argmax hits, counted rows, bad},
    lse f32 [n]) of cross-entropy over logits[rows] (csrc/fused.hip); no
    host sync."""
    n = labels.numel()
    dev = logits.device
    lse = torch.empty(max(1, n), dtype=torch.float32, device=dev)
    loss = torch.empty((), dtype=torch.float32, device=dev)
    counts = torch.empty(3, dtype=torch.int64, device=dev)
    wsb = int(L.load().grws_cross_entropy_workspace_bytes(n))
    ws = torch.empty(max(1, wsb), dtype=torch.uint8, device=dev)
    L.call("grws_cross_entropy_fwd", L.ptr(logits), L.dtype_code(logits.dtype), logits.stride(0),
           logits.shape[0], logits.shape[1], L.ptr(rows) if rows is not None else None, L.ptr(labels), n,
           L.ptr(lse), L.ptr(loss), L.ptr(counts), L.ptr(ws), wsb, L.stream_of(dev))
    return loss, counts, lse


def cross_entropy_bwd(logits: torch.Tensor, rows: Optional[torch.Tensor], labels: torch.Tensor,
                      lse: torch.Tensor, dloss: torch.Tensor, counts: torch.Tensor) -> torch.Tensor:
    """Gradient of cross_entropy_fwd's loss w.r.t. logits (zero outside rows),
    written into a line-pitched buffer (the backward SpMM and the weight
    gradient then read it without a widening copy)."""
    grad = line_pitched_empty(logits.shape[0], logits.shape[1], logits.dtype, logits.device, zero=True)
    dl = dloss.detach().float().reshape(1).contiguous()
    L.call("grws_cross_entropy_bwd", L.ptr(logits), L.dtype_code(logits.dtype), logits.stride(0),
           logits.shape[0], logits.shape[1], L.ptr(rows) if rows is not None else None, L.ptr(labels),
           labels.numel(), L.ptr(lse), L.ptr(dl), L.ptr(counts), L.ptr(grad), L.dtype_code(grad.dtype),
           grad.stride(0), L.stream_of(logits.device))
    return grad
