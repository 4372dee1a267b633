"""On-device COO -> CSR -> BCSR construction and the cached BCSR transpose.

Front end of the gfx950 builder kernels (csrc/bcsr_build.hip, C ABI in
include/grws.h).  Replaces, for graphs on the GPU:
  * BCSRGraph._coo_to_csr  (data/bcsr.py:162-187, torch argsort/bincount),
  * csr_to_bcsr_cpu        (core/wrapper/convert_wrapper.cpp:27-180, host
                            OpenMP, reached through data/bcsr.py:190-234),
and adds the BCSR of A^T that the backward pass multiplies with (the
reference scatters A^T G with atomics instead, spmm_tc.cuh:211-270).
Workspaces and outputs are torch tensors; the library allocates nothing.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from .core import _lib as L


def available() -> bool:
    """True when the loaded libgrws.so carries the device builder."""
    try:
        return hasattr(L.load(), "grws_bcsr_build_count")
    except ImportError:
        return False


def _i32(t: torch.Tensor, dev) -> torch.Tensor:
    return t.to(dev, torch.int32).contiguous()


def coo_to_csr_device(num_rows: int, num_cols: int, src: torch.Tensor, dst: torch.Tensor,
                      edge_weights: Optional[torch.Tensor] = None):
    """COO -> CSR on the device (data/bcsr.py:162-187): stable sort by
    (src, dst); returns (num_edges, row_ptr int64, col_idx int32, values f32)."""
    dev = src.device
    L.require_device("coo_to_csr_device", dev)  # the other inputs are moved to dev below
    s = _i32(src, dev)
    d = _i32(dst, dev)
    w = None if edge_weights is None else edge_weights.to(dev, torch.float32).contiguous()
    nnz = s.numel()
    row_ptr = torch.empty(num_rows + 1, dtype=torch.int64, device=dev)
    col_idx = torch.empty(max(nnz, 1), dtype=torch.int32, device=dev)
    values = torch.empty(max(nnz, 1), dtype=torch.float32, device=dev)
    wsb = int(L.load().grws_coo_to_csr_workspace_bytes(nnz, num_rows, num_cols))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    L.call("grws_coo_to_csr", L.ptr(s), L.ptr(d), L.ptr(w), nnz, num_rows, num_cols,
           L.ptr(row_ptr), L.ptr(col_idx), L.ptr(values), L.ptr(ws), wsb, L.stream_of(dev))
    return nnz, row_ptr, col_idx[:nnz], values[:nnz]


def _build(row_ptr, rows, cols, values, nnz: int, num_rows: int, num_cols: int, tile_cols: int,
           transpose: bool, values_dtype: torch.dtype, dev) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    R = num_cols if transpose else num_rows
    W = (R + 15) // 16
    win = torch.empty(W + 1, dtype=torch.int64, device=dev)
    wsb = int(L.load().grws_bcsr_build_workspace_bytes(nnz, num_rows, num_cols, int(transpose)))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    T = ctypes.c_int64()
    stream = L.stream_of(dev)
    L.call("grws_bcsr_build_count", L.ptr(row_ptr), L.ptr(rows), L.ptr(cols), L.ptr(values), nnz,
           num_rows, num_cols, tile_cols, int(transpose), L.ptr(win), L.ptr(ws), wsb,
           ctypes.byref(T), stream)
    T = T.value
    out_cols = torch.empty(T * tile_cols, dtype=torch.int32, device=dev)
    out_vals = torch.empty(T * 16 * tile_cols, dtype=values_dtype, device=dev)
    L.call("grws_bcsr_build_fill", nnz, num_rows, num_cols, tile_cols, int(transpose), L.ptr(win), T,
           L.ptr(out_cols), L.ptr(out_vals), L.dtype_code(values_dtype), L.ptr(ws), wsb, stream)
    return win, out_cols, out_vals


def csr_to_bcsr_device(num_rows: int, num_cols: int, row_ptr: torch.Tensor, col_idx: torch.Tensor,
                       values: Optional[torch.Tensor], tile_cols: int = 8,
                       values_dtype: torch.dtype = torch.float32, transpose: bool = False):
    """CSR -> BCSR on the device.  Same three arrays as csr_to_bcsr_cpu
    (convert_wrapper.cpp:27-180); values cast to `values_dtype` (round to
    nearest even).  transpose=True builds the BCSR of A^T."""
    dev = row_ptr.device
    L.require_device("csr_to_bcsr_device", dev)  # the other inputs are moved to dev below
    rp = row_ptr.to(dev, torch.int64).contiguous()
    ci = _i32(col_idx, dev)
    va = None if values is None else values.to(dev, torch.float32).contiguous()
    if rp.numel() != num_rows + 1:
        raise ValueError("row_ptr must have num_rows + 1 entries")
    return _build(rp, None, ci, va, ci.numel(), int(num_rows), int(num_cols), int(tile_cols),
                  transpose, values_dtype, dev)


def coo_to_bcsr_device(num_rows: int, num_cols: int, rows: torch.Tensor, cols: torch.Tensor,
                       values: Optional[torch.Tensor], tile_cols: int = 16,
                       values_dtype: torch.dtype = torch.float32, transpose: bool = False):
    """COO (any order, duplicates allowed: the last in input order wins) ->
    BCSR on the device, in one sort."""
    dev = rows.device
    L.require_device("coo_to_bcsr_device", dev)  # the other inputs are moved to dev below
    r = _i32(rows, dev)
    c = _i32(cols, dev)
    va = None if values is None else values.to(dev, torch.float32).contiguous()
    if r.numel() != c.numel():
        raise ValueError("rows and cols differ in length")
    return _build(None, r, c, va, r.numel(), int(num_rows), int(num_cols), int(tile_cols),
                  transpose, values_dtype, dev)


def bcsr_to_coo(window_offset: torch.Tensor, col_indices: torch.Tensor, values: torch.Tensor,
                tile_cols: int, num_cols: int):
    """Edges of a BCSR graph: every slot with a column in [0, num_cols) and a
    non-zero value.  Returns (rows int32, cols int32, values f32)."""
    dev = window_offset.device
    L.require_device("bcsr_to_coo", dev, window_offset, col_indices, values)
    if not (window_offset.is_contiguous() and col_indices.is_contiguous() and values.is_contiguous()):
        raise RuntimeError("bcsr_to_coo: the graph arrays must be contiguous")
    W = window_offset.numel() - 1
    T = col_indices.numel() // tile_cols
    view = L.BcsrView(L.ptr(window_offset), L.ptr(col_indices), L.ptr(values), W, T, 16, tile_cols,
                      L.dtype_code(values.dtype), 0)
    wsb = int(L.load().grws_bcsr_to_coo_workspace_bytes(T))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    n = ctypes.c_int64()
    stream = L.stream_of(dev)
    L.call("grws_bcsr_to_coo_count", ctypes.byref(view), num_cols, L.ptr(ws), wsb, ctypes.byref(n),
           stream)
    n = n.value
    rows = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    cols = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    vals = torch.empty(max(n, 1), dtype=torch.float32, device=dev)
    L.call("grws_bcsr_to_coo_fill", ctypes.byref(view), num_cols, L.ptr(rows), L.ptr(cols),
           L.ptr(vals), L.ptr(ws), wsb, stream)
    return rows[:n], cols[:n], vals[:n]


def transpose_arrays(window_offset: torch.Tensor, col_indices: torch.Tensor, values: torch.Tensor,
                     tile_cols: int, num_cols: int, out_tile_cols: Optional[int] = None):
    """BCSR arrays of A^T for a BCSR A with `num_cols` columns.  A^T has
    ceil(num_cols/16) windows; its columns are A's rows (0 .. 16W-1)."""
    W = window_offset.numel() - 1
    rows, cols, vals = bcsr_to_coo(window_offset, col_indices, values, tile_cols, num_cols)
    return coo_to_bcsr_device(16 * W, num_cols, rows, cols, vals,
                              tile_cols=out_tile_cols or tile_cols, values_dtype=values.dtype,
                              transpose=True)


def transpose(graph):
    """BCSRGraph of A^T (rows = graph.num_cols, cols = graph's 16W padded rows)."""
    from .data.bcsr import BCSRGraph
    win, cols, vals = transpose_arrays(graph.window_offset, graph.original_col_indices,
                                       graph.values_condensed, graph.tile_cols, graph.num_cols)
    AT = BCSRGraph(num_nodes=graph.num_cols, num_edges=graph.num_edges, tile_rows=16,
                   tile_cols=graph.tile_cols, window_offset=win, original_col_indices=cols,
                   values_condensed=vals, device=graph.window_offset.device,
                   num_rows=graph.num_cols, num_cols=16 * graph.num_windows,
                   values_dtype=graph.values_condensed.dtype)
    # the longest window (one sync, here rather than at the first product):
    # lets a small transpose (a sampled block's) skip the SpMM work plan
    if win.numel() > 1:
        AT.max_window_slabs = (int((win[1:] - win[:-1]).max().item()) * graph.tile_cols + 15) // 16
    return AT
