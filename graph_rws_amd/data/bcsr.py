"""BCSRGraph: the reference's BCSR container (data/bcsr.py:23-306) on MI355X.

Layout (unchanged, data/bcsr.py:24-33):
  window_offset        int64 [W+1]      prefix sum of tiles per 16-row window
  original_col_indices int32 [T*tc]     ascending unique global columns per
                                        window, -1 padding in the last tile
  values_condensed     [T*16*tc]        row-major [tile][row][col]

Differences from the reference, all opt-in or invisible to its callers:
  * `values_dtype` keyword: float32 (the reference's forced type, :50) by
    default; float16/bfloat16 halve the value bytes the SpMM streams;
  * graphs on a CUDA device are built by the gfx950 device builder when the
    library provides it, otherwise by the host converter (as the reference);
  * `spmm_plan()` caches the SpMM schedule, `transpose()` caches A^T (used
    by the backward pass instead of an atomic scatter).
"""
from __future__ import annotations

import weakref

from typing import Any, Dict, Optional

import numpy as np
import torch

from ..core import csr_to_bcsr_cpu, build_spmm_plan, default_slabs


def _placed(t: torch.Tensor, device, dtype: torch.dtype) -> torch.Tensor:
    """t on `device` with `dtype`: t itself when it already is (the common
    case of arrays made on the device, e.g. sampled blocks), else a copy."""
    if t.dtype == dtype and (device is None or t.device == device):
        return t
    return t.to(device, non_blocking=True).to(dtype)


class BCSRGraph:
    """BCSR graph (data/bcsr.py:23-62)."""

    def __init__(self,
                 num_nodes: int,
                 num_edges: int,
                 tile_rows: int,
                 tile_cols: int,
                 window_offset: torch.Tensor,
                 original_col_indices: torch.Tensor,
                 values_condensed: torch.Tensor,
                 device: Optional[torch.device] = None,
                 num_rows: Optional[int] = None,
                 num_cols: Optional[int] = None,
                 values_dtype: Optional[torch.dtype] = None) -> None:
        self.device = device
        vdt = torch.float32 if values_dtype is None else values_dtype
        self.window_offset = _placed(window_offset, device, torch.int64)
        self.original_col_indices = _placed(original_col_indices, device, torch.int32)
        self.values_condensed = _placed(values_condensed, device, vdt)
        self.num_rows = int(num_rows) if num_rows is not None else int(num_nodes)
        self.num_cols = int(num_cols) if num_cols is not None else int(num_nodes)
        self.num_nodes = int(num_nodes)
        self.num_edges = num_edges
        self.tile_rows = int(tile_rows)
        self.tile_cols = int(tile_cols)
        if self.tile_rows != 16:
            raise ValueError("tile_rows must be 16 (one row window)")
        self.num_windows = int(self.window_offset.shape[0] - 1)
        # set from the array sizes (the reference leaves it None, :62)
        self.num_tiles = int(self.original_col_indices.numel() // self.tile_cols)
        # SpMM plans and the transpose, shared by shallow copies (the model
        # copies the graph once per layer per forward, model.py:88-96)
        self._cache: Dict[Any, Any] = {}

    # ---------------- constructors (data/bcsr.py:65-159) ----------------

    # num_edges is an int, or a 0-dim device tensor counted on the stream
    # when the graph was made (from_components): it is read, and kept as an
    # int, on first access, so that building a sampled layer costs no host
    # sync unless its edge count is asked for
    @property
    def num_edges(self) -> int:
        n = self._num_edges
        if isinstance(n, torch.Tensor):
            n = self._num_edges = int(n.item())
        return n

    @num_edges.setter
    def num_edges(self, v) -> None:
        self._num_edges = v if isinstance(v, torch.Tensor) else int(v)

    @classmethod
    def from_dgl(cls, g: Any, tile_rows: int = 16, tile_cols: int = 8,
                 values_dtype: Optional[torch.dtype] = None) -> "BCSRGraph":
        """From a DGLGraph-like object (num_nodes(), edges(), edata, device)."""
        device = g.device
        num_nodes = g.num_nodes()
        src, dst = g.edges()
        edge_weights = g.edata.get("weight", None)
        num_edges, row_ptr, col_idx, values = cls._coo_to_csr(num_nodes, src, dst, edge_weights,
                                                              device, num_cols=num_nodes)
        return cls._from_csr(num_rows=num_nodes, row_ptr=row_ptr, col_idx=col_idx,
                             edge_values=values, tile_rows=tile_rows, tile_cols=tile_cols,
                             device=device, num_cols=num_nodes, values_dtype=values_dtype)

    @classmethod
    def from_mtx(cls, filepath: str, index_base: int = 0, undirected: bool = False,
                 tile_rows: int = 16, tile_cols: int = 8, device: Optional[torch.device] = None,
                 values_dtype: Optional[torch.dtype] = None) -> "BCSRGraph":
        """From a Matrix Market file (data/bcsr.py:90-131): all-ones values,
        square, duplicates summed by scipy's CSR constructor."""
        import scipy.io as sio
        import scipy.sparse as sps
        if device is None:
            device = torch.device("cuda" if torch.cuda.is_available() else "cpu")
        coo = sio.mmread(filepath).tocoo()
        rows = coo.row.astype(np.int64)
        cols = coo.col.astype(np.int64)
        if index_base == 1:
            rows -= 1
            cols -= 1
        if undirected:
            rows, cols = np.concatenate([rows, cols]), np.concatenate([cols, rows])
        num_rows = int(max(rows.max(), cols.max()) + 1)
        data = np.ones_like(rows, dtype=np.float32)
        csr = sps.csr_matrix((data, (rows, cols)), shape=(num_rows, num_rows))
        return cls._from_csr(num_rows=num_rows,
                             row_ptr=torch.from_numpy(csr.indptr.astype(np.int64)),
                             col_idx=torch.from_numpy(csr.indices.astype(np.int32)),
                             edge_values=torch.from_numpy(csr.data.astype(np.float32)),
                             tile_rows=tile_rows, tile_cols=tile_cols, device=device,
                             num_cols=num_rows, values_dtype=values_dtype)

    @classmethod
    def from_components(cls, window_offset: torch.Tensor, original_col_indices: torch.Tensor,
                        values_condensed: torch.Tensor, num_rows: int, num_cols: int,
                        tile_rows: int, tile_cols: int, device: Optional[torch.device] = None,
                        values_dtype: Optional[torch.dtype] = None) -> "BCSRGraph":
        """From kernel outputs (data/bcsr.py:134-159).  num_edges is the
        count of non-zero values, as in the reference (:147), counted on the
        values' stream now and read on first access."""
        if device is None:
            device = window_offset.device
        nnz = torch.count_nonzero(values_condensed) if values_condensed.numel() > 0 else 0
        return cls(num_nodes=int(num_rows), num_edges=nnz, tile_rows=tile_rows, tile_cols=tile_cols,
                   window_offset=window_offset, original_col_indices=original_col_indices,
                   values_condensed=values_condensed, device=device, num_rows=int(num_rows),
                   num_cols=int(num_cols),
                   values_dtype=values_dtype if values_dtype is not None else
                   (values_condensed.dtype if values_condensed.is_floating_point() else None))

    @classmethod
    def from_csr(cls, row_ptr: torch.Tensor, col_idx: torch.Tensor, values: Optional[torch.Tensor],
                 num_rows: int, num_cols: Optional[int] = None, tile_rows: int = 16,
                 tile_cols: int = 16, device: Optional[torch.device] = None,
                 values_dtype: Optional[torch.dtype] = None) -> "BCSRGraph":
        """From a CSR matrix (row_ptr int64 [n+1], col_idx int32, values)."""
        if device is None:
            device = row_ptr.device
        if values is None:
            values = torch.ones(col_idx.numel(), dtype=torch.float32, device=row_ptr.device)
        return cls._from_csr(num_rows=num_rows, row_ptr=row_ptr, col_idx=col_idx,
                             edge_values=values, tile_rows=tile_rows, tile_cols=tile_cols,
                             device=device, num_cols=num_cols, values_dtype=values_dtype)

    # ---------------- conversions (data/bcsr.py:162-234) ----------------
    @classmethod
    def _coo_to_csr(cls, num_rows: int, src: torch.Tensor, dst: torch.Tensor,
                    edge_weights: Optional[torch.Tensor], device: torch.device,
                    num_cols: Optional[int] = None):
        """COO -> CSR with torch ops (data/bcsr.py:163-187).  The sort key is
        row * num_cols + col (the reference multiplies by num_rows, :170,
        which misorders rectangular blocks); the sort is stable so duplicate
        edges keep their input order."""
        ncols = max(1, int(num_cols) if num_cols is not None else int(num_rows))
        from .. import builder
        if src.is_cuda and builder.available():
            num_edges, row_ptr, col_idx, values = builder.coo_to_csr_device(
                int(num_rows), ncols, src, dst, edge_weights)
            return num_edges, row_ptr.to(device), col_idx.to(device), values.to(device)
        sort_key = src.to(torch.long) * ncols + dst.to(torch.long)
        perm = torch.sort(sort_key, stable=True).indices
        src = src[perm]
        dst = dst[perm]
        num_edges = int(src.numel())
        if edge_weights is not None:
            values = edge_weights[perm].to(device).to(torch.float32)
        else:
            values = torch.ones(num_edges, dtype=torch.float32, device=device)
        row_counts = torch.bincount(src.to(torch.long), minlength=num_rows).to(torch.int64)
        row_ptr = torch.zeros(num_rows + 1, dtype=torch.int64, device=device)
        torch.cumsum(row_counts, dim=0, out=row_ptr[1:])
        col_idx = dst.to(torch.int32)
        return num_edges, row_ptr, col_idx, values

    @classmethod
    def _from_csr(cls, num_rows: int, row_ptr: torch.Tensor, col_idx: torch.Tensor,
                  edge_values: torch.Tensor, tile_rows: int, tile_cols: int, device: torch.device,
                  num_cols: Optional[int] = None,
                  values_dtype: Optional[torch.dtype] = None) -> "BCSRGraph":
        """CSR -> BCSR (data/bcsr.py:190-234)."""
        if num_cols is None:
            num_cols = num_rows
        device = torch.device(device) if device is not None else row_ptr.device
        from .. import builder
        if device.type == "cuda" and builder.available():
            win, cols, vals = builder.csr_to_bcsr_device(
                int(num_rows), int(num_cols), row_ptr.to(device), col_idx.to(device),
                edge_values.to(device), tile_cols=tile_cols,
                values_dtype=values_dtype or torch.float32)
        else:
            win, cols, vals = csr_to_bcsr_cpu(int(num_rows), row_ptr.to("cpu", torch.int64),
                                              col_idx.to("cpu", torch.int32),
                                              edge_values.to("cpu", torch.float32),
                                              int(tile_rows), int(tile_cols))
        return cls(num_nodes=int(num_rows), num_edges=int(col_idx.numel()), tile_rows=tile_rows,
                   tile_cols=tile_cols, window_offset=win.to(device),
                   original_col_indices=cols.to(device), values_condensed=vals.to(device),
                   device=device, num_rows=int(num_rows), num_cols=int(num_cols),
                   values_dtype=values_dtype)

    # ---------------- utilities ----------------
    def to(self, device: torch.device, non_blocking: bool = False) -> "BCSRGraph":
        """Move to a device, keeping the rectangular shape (data/bcsr.py:238-258)."""
        if device == self.device:
            return self
        return BCSRGraph(num_nodes=self.num_rows, num_edges=self._num_edges,
                         tile_rows=self.tile_rows, tile_cols=self.tile_cols,
                         window_offset=self.window_offset.to(device, non_blocking=non_blocking),
                         original_col_indices=self.original_col_indices.to(device, non_blocking=non_blocking),
                         values_condensed=self.values_condensed.to(device, non_blocking=non_blocking),
                         device=device, num_rows=self.num_rows, num_cols=self.num_cols,
                         values_dtype=self.values_condensed.dtype)

    def with_values_dtype(self, dtype: torch.dtype) -> "BCSRGraph":
        """Same structure, values cast to `dtype` (round to nearest even)."""
        return BCSRGraph(num_nodes=self.num_rows, num_edges=self._num_edges,
                         tile_rows=self.tile_rows, tile_cols=self.tile_cols,
                         window_offset=self.window_offset,
                         original_col_indices=self.original_col_indices,
                         values_condensed=self.values_condensed, device=self.device,
                         num_rows=self.num_rows, num_cols=self.num_cols, values_dtype=dtype)

    def __repr__(self) -> str:
        return (f"BCSRGraph(rows={self.num_rows}, cols={self.num_cols}, windows={self.num_windows}, "
                f"tiles={self.num_tiles}, tile={self.tile_rows}x{self.tile_cols}, "
                f"values={self.values_condensed.dtype}, device={self.device})")

    @classmethod
    def from_dgl_block(cls, block: Any, tile_rows: int = 16, tile_cols: int = 8,
                       values_dtype: Optional[torch.dtype] = None) -> "BCSRGraph":
        """A DGL message-flow block (dst rows x src cols, data/bcsr.py:266-306)."""
        device = block.device
        num_rows = block.num_dst_nodes()
        num_cols = block.num_src_nodes()
        src, dst = block.edges()
        edge_weights = block.edata.get("weight", None) if "weight" in block.edata else None
        num_edges, row_ptr, col_idx, values = cls._coo_to_csr(num_rows, dst, src, edge_weights,
                                                              device, num_cols=num_cols)
        return cls._from_csr(num_rows=num_rows, row_ptr=row_ptr, col_idx=col_idx,
                             edge_values=values, tile_rows=tile_rows, tile_cols=tile_cols,
                             device=device, num_cols=num_cols, values_dtype=values_dtype)

    # ---------------- MI355X additions ----------------
    def spmm_plan(self, n_cols: int):
        """Cached SpMM schedule for outputs of width n_cols, or None when no
        window can exceed the per-item slab budget (``max_window_slabs``
        known, e.g. for sampled blocks): then one work item per window is the
        schedule and no plan needs building.  A graph whose arrays are
        refilled in place between replays of a captured step
        (``refilled = True``) never takes a plan: its windows change under
        the plan."""
        if getattr(self, "refilled", False):
            return None
        slabs = default_slabs(self.num_windows, self.num_tiles, self.tile_cols, n_cols)
        mws = getattr(self, "max_window_slabs", None)
        if mws is not None and mws <= slabs:
            return None
        from ..core.ops import TensorKey
        ent = self._cache.get(("plan", slabs))
        if ent is None or not ent[0].matches((self.window_offset,), (self.num_tiles, self.tile_cols)):
            p = build_spmm_plan(self.window_offset, self.num_tiles, self.tile_cols, slabs)
            ent = (TensorKey((self.window_offset,), (self.num_tiles, self.tile_cols)), p)
            self._cache[("plan", slabs)] = ent
        return ent[1]

    def packed_tiles(self):
        """The packed copy of the values the SpMM reads instead of the dense
        tiles (16x16 tiles of f16/bf16 values), built on this graph's second
        SpMM and kept while the value and column arrays are unchanged.  A
        graph multiplied once (a sampled block) is never packed: packing reads
        the dense values twice, so it pays only from the second product on.
        None when packing is off or does not apply."""
        from ..core import ops as _ops
        if not _ops.PACK_TILES or self.tile_cols != 16 or getattr(self, "refilled", False):
            return None
        from ..core.ops import TensorKey
        v, c = self.values_condensed, self.original_col_indices
        ent = self._cache.get("packed")
        if ent is None or not ent[0].matches((v, c)):
            self._cache["packed"] = (TensorKey((v, c)), 1, None)
            return None
        key, calls, p = ent
        if p is None and calls == 1:
            p = _ops.pack_tiles(self.window_offset, c, v, self.tile_cols) or False
            self._cache["packed"] = (key, 2, p)
        return p or None

    def grouped_tiles(self, num_cols: int, n_cols: int = 0):
        """Grouped tiles (windows sharing their union columns, see
        core.ops.group_tiles) for products over num_cols X rows, built on
        this graph's second such product (with the group size that suits
        that product's width n_cols, core.ops.group_size_for) and kept while
        the arrays are unchanged; None when grouping is off, does not apply,
        or would not pay on this graph (decided once per graph state).

        One layout is cached per group size: products of different widths
        that want different group sizes (the 608-column features and the
        256-column hidden layers) each get their own, built on the second
        product of that group size."""
        from ..core import ops as _ops
        if (not _ops.GROUPED or not _ops.PACK_TILES or getattr(self, "refilled", False)
                or self.values_condensed.dtype not in (torch.float16, torch.bfloat16)):
            return None
        from ..core.ops import TensorKey
        gs = int(_ops.group_size_for(n_cols))
        arrays = (self.window_offset, self.original_col_indices, self.values_condensed)
        slot = ("grouped", gs)
        ent = self._cache.get(slot)
        if ent is None or not ent[0].matches(arrays, (int(num_cols),)):
            self._cache[slot] = (TensorKey(arrays, (int(num_cols),)), 1, None)
            return None
        key, calls, g = ent
        if g is None and calls == 1:
            g = _ops.group_tiles(self.window_offset, self.original_col_indices, self.values_condensed,
                                 self.tile_cols, int(num_cols), group_size=gs) or False
            self._cache[slot] = (key, 2, g)
        return g or None

    def _gather_input(self, x: torch.Tensor) -> torch.Tensor:
        """x, or a copy whose rows start on 128-byte lines when x's row pitch
        is not a multiple of 128 bytes and this graph gathers every row many
        times (at least 8 column slots per row of x): a 224-byte row at a
        224-byte pitch straddles lines, and the SpMM gathering such rows ran
        19% slower (c4, 112 columns).  Each input's copy is kept while that
        input is alive and unmodified, and dropped when it dies: the layer-0
        features of full-graph training are copied once, although the same
        graph multiplies other (short-lived) inputs in between.

        While the current stream is being captured the cache is bypassed:
        the copy is made afresh, so its kernel is recorded in the graph and
        every replay re-reads x (a replay after ``x.copy_(new)`` multiplies
        the new values, not the copy made before the capture)."""
        esz = x.element_size()
        if (x.dim() != 2 or x.stride(1) != 1 or (x.stride(0) * esz) % 128 == 0
                or x.shape[1] * esz < 64 or self.num_tiles * self.tile_cols < 8 * x.shape[0]):
            return x
        if x.is_cuda and torch.cuda.is_current_stream_capturing():
            from .layout import aligned_rows
            return aligned_rows(x.detach())
        copies = self._cache.setdefault("aligned_x", {})
        key = id(x)
        ent = copies.get(key)
        if ent is not None and ent[0]() is x and ent[1] == x._version:
            return ent[2]
        from .layout import aligned_rows
        xa = aligned_rows(x.detach())

        def _drop(ref, copies=copies, key=key):
            if copies.get(key, (None,))[0] is ref:
                del copies[key]

        copies[key] = (weakref.ref(x, _drop), x._version, xa)
        return xa

    def padded_input(self, x: torch.Tensor) -> Optional[torch.Tensor]:
        """The line-aligned copy this graph gathers x through, with its
        zero padding columns ([rows, pitch], pitch a multiple of 128 bytes),
        or None when x is gathered as it is.  Products over the padded
        width equal those over x plus exact zeros."""
        xa = self._gather_input(x)
        if xa is x or xa.stride(0) <= xa.shape[1]:
            return None
        return xa.as_strided((xa.shape[0], xa.stride(0)), (xa.stride(0), 1))

    def spmm(self, x: torch.Tensor, out: Optional[torch.Tensor] = None,
             residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Y[16W, N] = A x on the device (columns >= x.shape[0] contribute
        nothing); plus residual on its rows when given (Y = A x + R there)."""
        from ..core import spmm as _spmm
        x = self._gather_input(x)
        same = x.dtype == self.values_condensed.dtype
        from ..core import ops as _ops
        grouped = (self.grouped_tiles(x.shape[0], x.shape[1])
                   if _ops.grouped_supported(x, self.values_condensed) and x.shape[1] >= _ops.GROUP_MIN_N else None)
        return _spmm(self.window_offset, self.original_col_indices, self.values_condensed, x,
                     self.tile_cols, plan=None if grouped is not None else self.spmm_plan(x.shape[1]), out=out,
                     packed=self.packed_tiles() if same and grouped is None else None,
                     max_window_slabs=getattr(self, "max_window_slabs", None) or 0, residual=residual,
                     grouped=grouped)

    def transpose(self) -> "BCSRGraph":
        """Cached BCSR of A^T (num_cols x 16W), built on the device.  Rebuilt
        when the column or value arrays are replaced or modified in place."""
        from ..core.ops import TensorKey
        arrays = (self.window_offset, self.original_col_indices, self.values_condensed)
        t = self._cache.get("T")
        if t is None or not t[0].matches(arrays, (self.num_cols,)):
            key = TensorKey(arrays, (self.num_cols,))
            from .. import builder
            t = (key, builder.transpose(self))
            self._cache["T"] = t
        return t[1]

    def spmm_transpose(self, grad_out: torch.Tensor, num_cols: Optional[int] = None) -> torch.Tensor:
        """A^T grad_out, [num_cols, D] (core_lib.spmm_transpose semantics,
        spmm_wrapper.cu:109-152), as a forward SpMM over the cached A^T:
        deterministic, no atomics.  grad_out: [16W, D]."""
        n = self.num_cols if num_cols is None else int(num_cols)
        AT = self.transpose()
        Y = AT.spmm(grad_out)
        if Y.shape[0] >= n:
            return Y[:n]
        return torch.nn.functional.pad(Y, (0, 0, 0, n - Y.shape[0]))
