"""BCSRSampler: the reference's window top-K multi-layer sampler
(sampler/sampler.py:31-307) over the gfx950 kernels of
csrc/window_sample.hip.

Same constructor arguments, same ``sample_layers(g, seed_nodes)`` contract:
one BCSRGraph per model layer, input side first.  Hop 0 runs from the seeds
with the LAST fanout (``reversed(fanouts)``, sampler.py:204).  Each layer
has ``num_rows = 16 * len(active_windows)`` and ``num_cols = g.num_cols``,
and carries ``active_windows`` / ``active_masks``, which the model's reindex
uses (models/model.py:126-143).  Column ids are global.

``repack_subgraph`` (sampler.py:420-690) repacks a window set into a halo
graph on the device (csrc/repack.hip).
"""
from __future__ import annotations

from typing import List

import torch

from ..core import sample_all_layers
from ..core.ops import CapturedWindowSampler, SampleState, TensorKey, repack
from ..data import BCSRGraph


class BCSRSampler:
    def __init__(self, fanouts: List[int], tile_rows: int = 16, tile_cols: int = 8,
                 warps_per_block: int = 8, partition_book: list = None, verbose: bool = True,
                 static_scores: torch.Tensor = None, window_part_ids: torch.Tensor = None,
                 part_ranges: torch.Tensor = None, hacs_enabled: bool = False,
                 alpha: float = 1.0, beta: float = 10.0, delta: float = 0.0,
                 gamma_bonus: float = 0.0, score_scale: float = 100.0,
                 locality_enabled: bool = False, capture: bool = False):
        self.fanouts = list(fanouts)
        self.tile_rows = tile_rows
        self.tile_cols = tile_cols
        self.warps_per_block = warps_per_block
        self.partition_book = partition_book
        self.verbose = verbose
        self.time_tracker = {}
        self.static_scores = static_scores
        self.window_part_ids = window_part_ids
        self.part_ranges = part_ranges
        self.hacs_enabled = bool(hacs_enabled)
        self.locality_enabled = bool(locality_enabled)
        self.alpha = float(alpha)
        self.beta = float(beta)
        self.delta = float(delta)
        self.gamma_bonus = float(gamma_bonus)
        self.score_scale = float(score_scale)
        # not in the reference: replay every batch's call from a HIP graph
        # (CapturedWindowSampler, one per seed-count bucket), the same layers
        # bit for bit; phase timings are not recorded then
        self.capture = bool(capture)
        self._captures = {}

    def _hacs_args(self, device):
        """(static_scores, window_part_ids, part_starts, part_ends, use_hacs,
        locality) as the reference prepares them (sampler.py:101-151)."""
        use_hacs = self.hacs_enabled and self.static_scores is not None
        if not use_hacs:
            return None, None, None, None, 0, 0
        ss = torch.as_tensor(self.static_scores).to(device, torch.float32).contiguous()
        loc = int(self.locality_enabled and self.window_part_ids is not None
                  and self.part_ranges is not None)
        if not loc:
            return ss, None, None, None, 1, 0
        wp = torch.as_tensor(self.window_part_ids).to(device, torch.int32).contiguous()
        pr = torch.as_tensor(self.part_ranges).to(device, torch.int32)
        return ss, wp, pr[:, 0].contiguous(), pr[:, 1].contiguous(), 1, 1

    def sample_layers(self, g: BCSRGraph, seed_nodes: torch.Tensor) -> List[BCSRGraph]:
        """Samples len(fanouts) layers from `seed_nodes` (global node ids)."""
        device = g.window_offset.device if g.window_offset.is_cuda else torch.device("cuda")
        seeds = torch.as_tensor(seed_nodes).to(device, torch.int32).contiguous()
        if self.capture:
            if self.tile_rows != 16 or self.tile_cols not in (8, 16):
                raise RuntimeError("sample_all_layers supports 16x8 tiles (the reference's) and 16x16")
            if self.warps_per_block not in (4, 8):
                raise RuntimeError(f"Unsupported warps_per_block: {self.warps_per_block}. Only 4 and 8 allowed.")
            return self._build_layers(g, self._captured(g, seeds, device).run(seeds))
        ss, wp, ps, pe, use_hacs, loc = self._hacs_args(device)
        layers_data, timings = sample_all_layers(
            g.window_offset, g.original_col_indices, g.values_condensed, seeds,
            list(reversed(self.fanouts)), int(g.num_nodes), ss, wp, ps, pe, self.alpha, self.beta,
            self.delta, self.gamma_bonus, self.score_scale, use_hacs, loc, self.tile_rows,
            self.tile_cols, self.warps_per_block, with_timings=self.verbose)
        if self.verbose:
            n = len(self.fanouts)
            for i, t in enumerate(timings):
                st = self.time_tracker.setdefault(n - 1 - i, {"count": 0, "p1_sample": 0.0,
                                                              "p2_map": 0.0, "p3_recomp": 0.0,
                                                              "total": 0.0})
                st["count"] += 1
                st["p1_sample"] += t.phase1_sampling_time
                st["p2_map"] += t.phase2_mapping_time
                st["p3_recomp"] += t.phase3_recompression_time
                st["total"] += t.total_time
        return self._build_layers(g, layers_data)

    # buckets of seed counts that share a capture, and at most this many
    # captures kept (the least recently used is dropped)
    CAPTURE_BUCKET = 256
    MAX_CAPTURES = 4

    def _captured(self, g: BCSRGraph, seeds: torch.Tensor, device) -> CapturedWindowSampler:
        """The capture that serves this graph, these settings and this seed
        count (made on first use, then kept while the graph arrays and the
        score tensors are the same objects, unmodified)."""
        cap = -(-max(1, int(seeds.numel())) // self.CAPTURE_BUCKET) * self.CAPTURE_BUCKET
        tensors = [g.window_offset, g.original_col_indices, g.values_condensed]
        tensors += [t for t in (self.static_scores, self.window_part_ids, self.part_ranges)
                    if isinstance(t, torch.Tensor)]
        extra = (tuple(self.fanouts), int(g.num_nodes), self.tile_cols, self.hacs_enabled, self.locality_enabled,
                 self.alpha, self.beta, self.delta, self.gamma_bonus, self.score_scale,
                 tuple(id(t) for t in (self.static_scores, self.window_part_ids, self.part_ranges)))
        ent = self._captures.pop(cap, None)
        if ent is None or not ent[0].matches(tensors, extra):
            if len(self._captures) >= self.MAX_CAPTURES:
                self._captures.pop(next(iter(self._captures)))
            ss, wp, ps, pe, use_hacs, loc = self._hacs_args(device)
            c = CapturedWindowSampler(g.window_offset, g.original_col_indices, g.values_condensed,
                                      list(reversed(self.fanouts)), int(g.num_nodes), cap, ss, wp, ps, pe,
                                      self.alpha, self.beta, self.delta, self.gamma_bonus, self.score_scale,
                                      use_hacs, loc, self.tile_cols)
            ent = (TensorKey(tensors, extra), c)
        self._captures[cap] = ent  # most recently used last
        return ent[1]

    def _build_layers(self, g: BCSRGraph, layers_data) -> List[BCSRGraph]:
        """One BCSRGraph per sampled layer, input side first."""
        layers: List[BCSRGraph] = []
        for win, cols, vals, act, msk in layers_data:
            sub = BCSRGraph.from_components(window_offset=win, original_col_indices=cols,
                                            values_condensed=vals,
                                            num_rows=int(act.numel()) * self.tile_rows,
                                            num_cols=g.num_cols, tile_rows=self.tile_rows,
                                            tile_cols=self.tile_cols, device=win.device)
            sub.active_windows = act
            sub.active_masks = msk
            layers.insert(0, sub)
        return layers

    # ------------------------------------------------------------------
    # halo-aware repack of a window set (sampler.py:420-690)
    # ------------------------------------------------------------------
    def _repack_state(self, num_nodes: int, device) -> SampleState:
        st = getattr(self, "_repack_state_cache", None)
        if st is None or st.num_nodes < num_nodes or st.node_map.device != torch.device(device):
            st = SampleState(num_nodes, device)
            self._repack_state_cache = st
        return st

    def repack_subgraph(self, g: BCSRGraph, window_ids: torch.Tensor, max_external_ratio: float = 5.0,
                        dry_run: bool = False, generator: torch.Generator = None):
        """The selected windows of ``g`` as a halo graph (sampler.py:420-690).

        Rows: the windows' nodes (``num_internal_nodes``, window order).
        Columns: those nodes first, then the external neighbours (halo) in
        ascending id -- all of them, or, when there are more than
        ``int(num_internal_nodes * max_external_ratio)``, a random subset of
        that size drawn as the reference draws it (one ``torch.randperm``
        on the device; ``generator`` defaults to the device's default
        generator).  Edges to dropped or invalid columns become -1 with zero
        values; if a value is NaN, every value goes through
        ``nan_to_num_(0.0)`` (after ``num_edges`` was counted), as in the
        reference.  ``subgraph.inner_graph`` masks every halo column too
        (``num_cols = num_internal_nodes``).  Attributes as in the reference:
        ``original_node_ids``, ``original_window_ids``, ``is_local_input``,
        ``num_internal_nodes``.  Column arrays are stored flat (the reference
        keeps a ``[tiles, tile_cols]`` view of the same values).

        Runs on the device kernels of csrc/repack.hip; ``g`` must be resident
        on ``window_ids``' device.  Duplicate window ids are an error (the
        reference's result is ill-defined for them)."""
        from types import SimpleNamespace
        device = window_ids.device
        window_ids, _ = torch.sort(window_ids)
        if window_ids.numel() > 0:
            valid = (window_ids >= 0) & (window_ids < g.num_windows)
            window_ids = window_ids[valid]
        num_windows = window_ids.size(0)
        if dry_run:
            off = g.window_offset
            ids = window_ids.to(off.device, torch.int64)
            lengths = off[ids + 1] - off[ids]
            total_tiles = int(lengths.sum().item()) if lengths.numel() > 0 else 0
            stub = SimpleNamespace()
            stub.original_window_ids = window_ids
            stub.num_internal_nodes = num_windows * self.tile_rows
            stub.total_tiles = total_tiles
            stub.approx_values = total_tiles * self.tile_rows * self.tile_cols
            stub.approx_cols = total_tiles * self.tile_cols
            stub.values_condensed = None
            stub.original_col_indices = None
            return stub
        if g.tile_rows != self.tile_rows or g.tile_cols != self.tile_cols:
            raise ValueError(f"repack_subgraph: graph tiles {g.tile_rows}x{g.tile_cols} differ from the "
                             f"sampler's {self.tile_rows}x{self.tile_cols}")
        if g.window_offset.device != device:
            raise RuntimeError("repack_subgraph: the graph must be resident on the window ids' device")
        if num_windows > 1 and bool((window_ids[1:] == window_ids[:-1]).any()):
            raise ValueError("repack_subgraph: duplicate window ids")
        st = self._repack_state(g.num_nodes, device)
        r = repack(g.window_offset, g.original_col_indices, g.values_condensed, g.tile_cols, g.num_nodes,
                   window_ids, max_external_ratio, st, generator=generator)
        n_in = r.input_nodes.numel()
        subgraph = BCSRGraph.from_components(
            window_offset=r.window_offset, original_col_indices=r.halo_cols, values_condensed=r.halo_values,
            num_rows=r.num_internal, num_cols=n_in, tile_rows=self.tile_rows, tile_cols=self.tile_cols,
            device=device)
        subgraph.original_node_ids = r.input_nodes
        subgraph.original_window_ids = window_ids
        subgraph.is_local_input = True
        subgraph.num_internal_nodes = r.num_internal
        inner_vals = r.inner_values
        if r.any_nan:
            # in place: the halo graph holds the same tensor
            subgraph.values_condensed.nan_to_num_(0.0)
            inner_vals = subgraph.values_condensed.clone()
            T = r.inner_cols.numel() // self.tile_cols
            m = (r.inner_cols == -1).view(T, 1, self.tile_cols).expand(-1, self.tile_rows, -1)
            inner_vals.view(T, self.tile_rows, self.tile_cols).masked_fill_(m, 0.0)
        subgraph.inner_graph = BCSRGraph.from_components(
            window_offset=r.window_offset, original_col_indices=r.inner_cols, values_condensed=inner_vals,
            num_rows=r.num_internal, num_cols=r.num_internal, tile_rows=self.tile_rows,
            tile_cols=self.tile_cols, device=device)
        return subgraph

    def print_avg_timing(self):
        print("\n" + "-" * 60)
        print(" [Average Sampling Performance Summary (All Epochs)]")
        print("-" * 60)
        for layer_id in sorted(self.time_tracker):
            st = self.time_tracker[layer_id]
            c = st["count"]
            if c == 0:
                continue
            print(f"  [Layer {layer_id}] select {st['p1_sample'] / c:8.3f} ms | "
                  f"map {st['p2_map'] / c:8.3f} ms | recompress {st['p3_recomp'] / c:8.3f} ms | "
                  f"total {st['total'] / c:8.3f} ms")

    def __repr__(self):
        # the reference reads a missing self._bcsr_cache here (sampler.py:281-284)
        return (f"BCSRSampler(fanouts={self.fanouts}, tile={self.tile_rows}x{self.tile_cols}, "
                f"warps_per_block={self.warps_per_block})")
