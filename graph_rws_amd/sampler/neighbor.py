"""Node-wise fanout sampler on MI355X: Philox draws, unique + relabel, and a
BCSR block per hop.

Returns the same ``List[BCSRGraph]`` the reference's
``BCSRSampler.sample_layers`` returns (sampler/sampler.py:186-279): one
graph per model layer, input side first, hop 0 (from the seeds) drawn with
the LAST fanout as the reference does (``reversed(fanouts)``,
sampler.py:204).  Each graph is a message-flow block in the layout of
``BCSRGraph.from_dgl_block`` (data/bcsr.py:266-306): rows are the hop's
destination nodes, columns its source nodes, and the destination nodes are
the first columns ("target-top", layers/layer.py:159-161), so a layer's
self path is ``features[:num_rows]``.

Per hop, on the device (csrc/sample.hip, csrc/bcsr_build.hip):
  1. sampling  -- min(deg, k) distinct neighbours per frontier node, Floyd
                  over Philox4x32-10(seed, node, draw);
  2. relabel   -- frontier keeps [0, F), new sources appended in ascending
                  global id; the next frontier;
  3. BCSR      -- rows = destination positions, columns = source local ids,
                  values 1/sqrt((deg_u+1)(deg_v+1)) from full-graph
                  out-degrees.
The fused path runs every hop of the batch in one grws_sample_blocks call
with one stream sync; fused=False runs grws_sample_hop, grws_relabel and the
COO build per hop.  capture=True replays the fused call from a HIP graph
captured once per batch shape (seed counts bucketed by 64), which removes
the host's ~50 kernel launches per batch; the blocks are the same, bit for
bit.
"""
from __future__ import annotations

import time
from typing import List, Sequence

import torch

from ..core import relabel, sample_hop
from ..core.ops import CapturedSampleBlocks, SampleState, sample_blocks
from ..data import BCSRGraph


class NeighborSampler:
    """Fixed-fanout node-wise sampler over a CSR graph resident in HBM.

    Args:
        fanouts: neighbours per node for each model layer, input side first
            (as the reference's ``BCSRSampler(fanouts=...)``); each in [1, 64].
        seed: Philox key (the stream is counter = (node, draw)).
        tile_cols: 16 (MFMA-native) or 8 (the reference's tile).
        values_dtype: dtype of the blocks' values_condensed.
        capture: replay each batch from a HIP graph (fused path; one capture
            per CSR graph, transposes flags and bucket of 64 seed counts).
    """

    # captured batch shapes kept per sampler (least recently used dropped)
    MAX_CAPTURES = 8

    def __init__(self, fanouts: Sequence[int], seed: int = 42, tile_rows: int = 16,
                 tile_cols: int = 16, values_dtype: torch.dtype = torch.float32,
                 verbose: bool = False, fused: bool = True, capture: bool = False):
        if tile_rows != 16:
            raise ValueError("tile_rows must be 16")
        if tile_cols not in (8, 16):
            raise ValueError("tile_cols must be 8 or 16")
        for f in fanouts:
            if not 1 <= int(f) <= 64:
                raise ValueError(f"fanout {f} outside [1, 64]")
        self.fanouts = [int(f) for f in fanouts]
        self.seed = int(seed)
        self.tile_rows = 16
        self.tile_cols = int(tile_cols)
        self.values_dtype = values_dtype
        self.verbose = verbose
        self.last_stats: dict = {}
        self.total_edges = 0
        self.total_batches = 0
        # fused: the whole batch in one grws_sample_blocks call (dense relabel
        # state kept per graph, one sync); otherwise sample_hop + relabel +
        # COO build per hop
        self.fused = bool(fused)
        self.capture = bool(capture) and self.fused
        self._state = None
        self._captures: dict = {}

    def sample_layers(self, indptr: torch.Tensor, indices: torch.Tensor,
                      seed_nodes: torch.Tensor, transposes=None) -> List[BCSRGraph]:
        """Samples len(fanouts) hops from `seed_nodes` (distinct global ids).

        transposes: per layer (input side first), whether to build the
        block's transpose as well, in the same device call (fused path): the
        block's ``transpose()`` then returns it without a build.

        Every returned block carries ``src_nodes`` (int64 global ids of its
        columns, destination nodes first), ``num_sampled_edges`` and
        ``fanout``.  ``layers[0].src_nodes`` are the input nodes whose
        features the first layer reads."""
        from .. import builder
        dev = indptr.device
        num_nodes = indptr.numel() - 1
        frontier = seed_nodes.to(dev, torch.int64).contiguous()
        blocks: List[BCSRGraph] = []
        t0 = time.perf_counter()
        edges = 0
        if self.fused and (self._state is None or self._state.num_nodes != num_nodes
                           or self._state.node_map.device != dev):
            self._state = SampleState(num_nodes, dev)
        hop_fanouts = list(reversed(self.fanouts))
        hop_t = None
        if transposes is not None and self.fused:
            if len(transposes) != len(self.fanouts):
                raise ValueError("sample_layers: one transposes flag per layer")
            hop_t = [bool(t) for t in reversed(list(transposes))]
            if not any(hop_t):
                hop_t = None
        batch = None
        if self.capture and frontier.numel() > 0:
            batch = self._captured(indptr, indices, hop_fanouts, hop_t, frontier.numel()).run(frontier)
        elif self.fused:
            batch = sample_blocks(indptr, indices, frontier, hop_fanouts, self._state, seed=self.seed,
                                  tile_cols=self.tile_cols, values_dtype=self.values_dtype, transposes=hop_t)
        for h, k in enumerate(hop_fanouts):
            tr = None
            if self.fused:
                win, cols, vals, nxt, E = batch[h][:5]
                if hop_t is not None:
                    tr = batch[h][5]
            else:
                dst, src, val = sample_hop(indptr, indices, frontier, k, seed=self.seed)
                src_local, nxt = relabel(frontier, src, num_nodes)
                win, cols, vals = builder.coo_to_bcsr_device(
                    frontier.numel(), nxt.numel(), dst, src_local, val, tile_cols=self.tile_cols,
                    values_dtype=self.values_dtype)
                E = int(dst.numel())
            F, S = frontier.numel(), nxt.numel()
            g = BCSRGraph(num_nodes=F, num_edges=E, tile_rows=16,
                          tile_cols=self.tile_cols, window_offset=win, original_col_indices=cols,
                          values_condensed=vals, device=dev, num_rows=F, num_cols=S,
                          values_dtype=self.values_dtype)
            g.src_nodes = nxt
            g.dst_nodes = frontier
            g.num_sampled_edges = E
            # columns are local ids into the layer input (-1 only as padding):
            # the model needs no masking or reindex for this block
            g.columns_local = True
            # at most 16 x fanout distinct columns per window
            g.max_window_slabs = (16 * k + 15) // 16
            g.fanout = k
            if tr is not None:
                from ..core.ops import TensorKey
                twin, tcols, tvals, tmax = tr
                AT = BCSRGraph(num_nodes=S, num_edges=E, tile_rows=16, tile_cols=self.tile_cols,
                               window_offset=twin, original_col_indices=tcols, values_condensed=tvals,
                               device=dev, num_rows=S, num_cols=16 * g.num_windows, values_dtype=self.values_dtype)
                AT.max_window_slabs = (tmax * self.tile_cols + 15) // 16
                g._cache["T"] = (TensorKey((g.window_offset, g.original_col_indices, g.values_condensed),
                                           (g.num_cols,)), AT)
            blocks.insert(0, g)
            edges += g.num_sampled_edges
            frontier = nxt
        self.last_stats = {"edges": edges, "seconds": time.perf_counter() - t0,
                           "input_nodes": int(frontier.numel())}
        self.total_edges += edges
        self.total_batches += 1
        if self.verbose:
            s = self.last_stats
            print(f"[NeighborSampler] {len(self.fanouts)} hops, {s['edges']} edges, "
                  f"{s['input_nodes']} input nodes, {1e3 * s['seconds']:.3f} ms")
        return blocks

    def _captured(self, indptr, indices, hop_fanouts, hop_t, num_seeds: int) -> CapturedSampleBlocks:
        """The captured batch of this shape (created on first use)."""
        cap = -(-int(num_seeds) // 64) * 64
        key = (indptr.data_ptr(), indices.data_ptr(), indptr.numel(), indices.numel(), tuple(hop_fanouts),
               tuple(hop_t) if hop_t is not None else None, cap, self._state.node_map.data_ptr())
        c = self._captures.pop(key, None)
        if c is None:
            if len(self._captures) >= self.MAX_CAPTURES:
                self._captures.pop(next(iter(self._captures)))
            c = CapturedSampleBlocks(indptr, indices, hop_fanouts, self._state, self.seed, self.tile_cols,
                                     self.values_dtype, hop_t, cap)
        self._captures[key] = c  # most recently used last
        return c

    def __repr__(self) -> str:
        return (f"NeighborSampler(fanouts={self.fanouts}, seed={self.seed}, "
                f"tile={self.tile_rows}x{self.tile_cols}, values={self.values_dtype})")
