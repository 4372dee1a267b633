"""Full-graph training step replayed from a captured HIP graph.

``train_epoch_full`` (engine.py:44-83 of the reference) issues every kernel
of the step from Python: forward, cross-entropy, backward, gradient clipping
and Adam.  On a small graph (c1: 2,708 nodes, about 90 kernels of a few
microseconds each) the step is the host launching them.  ``GraphedFullStep``
records the step once on a HIP graph (``torch.cuda.graph``) and replays it:
the same kernels on the same buffers, with the host out of the loop.

Conditions, checked or established at construction:

* the optimizer updates on the device without host syncs: an optimizer
  built with ``capturable=True`` (torch's Adam / AdamW);
* the warm-up steps (on a side stream, default priority) build everything
  the graph keeps between calls: SpMM plans, packed tiles, the transpose, the
  masked layer-0 columns.  The captured step then issues no host sync and
  allocates only from the graph's pool.  The features' line-aligned copy
  (made when their row pitch straddles cache lines) is not taken from the
  cache under capture: its copy kernel is recorded, so every replay reads
  the features as they are then;
* dropout draws its seed on the device while the stream is captured, so each
  replay trains with a new mask.

A replay reads the tensors given at construction: update features, labels
or the training rows in place (``copy_``) to train on new values; new
tensors, new shapes or a modified graph need a new capture.  Training rows
updated in place must stay strictly ascending: the fused loss that the
capture recorded was chosen for distinct rows, and it writes (does not add)
each row's gradient, so a repeated row would get the gradient of one
occurrence only.  Parameters and
optimizer state are updated in place by every replay, as by the eager step.
"""
from __future__ import annotations

from typing import Optional

import torch

from .engine import train_epoch_full


class GraphedFullStep:
    def __init__(self, model, graphs_for_model, features: torch.Tensor, labels: torch.Tensor,
                 train_idx: torch.Tensor, optimizer: torch.optim.Optimizer, device,
                 warmup: int = 3, autocast_dtype: Optional[torch.dtype] = None):
        if not optimizer.defaults.get("capturable", False):
            raise ValueError("GraphedFullStep needs an optimizer that steps on the device: build it "
                             "with capturable=True (e.g. torch.optim.Adam(params, capturable=True))")
        self._args = (model, graphs_for_model, features, labels, train_idx, optimizer, device)
        self._dtype = autocast_dtype
        cur = torch.cuda.current_stream(device)
        side = torch.cuda.Stream(device)
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            for _ in range(max(2, int(warmup))):  # the second product packs the tiles
                self._step()
        cur.wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, capture_error_mode="thread_local"):
            self.loss, self.acc = self._step()
        self._idx_version = train_idx._version

    def _step(self):
        model, graphs, x, y, idx, opt, dev = self._args
        if self._dtype is None:
            return train_epoch_full(model, graphs, x, y, idx, opt, dev, sync=False)
        with torch.autocast("cuda", dtype=self._dtype):
            return train_epoch_full(model, graphs, x, y, idx, opt, dev, sync=False)

    def __call__(self):
        """One training step; returns (loss, accuracy) as device tensors that
        the next replay overwrites.  Training rows changed in place since the
        last call are checked first (one device reduction and one sync per
        change): they must still be strictly ascending."""
        idx = self._args[4]
        if idx._version != self._idx_version:
            from ..layers.fused import rows_distinct
            if not rows_distinct(idx):
                raise ValueError("GraphedFullStep: the training rows were updated in place to values that are "
                                 "not strictly ascending; the captured loss needs distinct rows (capture anew)")
            self._idx_version = idx._version
        self.graph.replay()
        return self.loss, self.acc


# ---------------------------------------------------------------------------
# mini-batch step over sampled blocks (helper/engine.py:86-256 of the reference)
# ---------------------------------------------------------------------------
def bucket_rows(x: int, floor: int = 256) -> int:
    """x rounded up to a step of 1/16 to 1/8 of its size, at least `floor`
    (a multiple of 16 rows): batches of nearly the same shape share a bucket."""
    if x <= floor:
        return floor
    step = max(floor, 1 << max(0, x.bit_length() - 4))
    return -(-x // step) * step


def _bcsr_buffers(rows, cols, windows, tiles, tc, vdt, device, flag):
    from ..data import BCSRGraph
    g = BCSRGraph(num_nodes=rows, num_edges=0, tile_rows=16, tile_cols=tc,
                  window_offset=torch.zeros(windows + 1, dtype=torch.int64, device=device),
                  original_col_indices=torch.full((tiles * tc,), -1, dtype=torch.int32, device=device),
                  values_condensed=torch.zeros(tiles * 16 * tc, dtype=vdt, device=device),
                  device=device, num_rows=rows, num_cols=cols, values_dtype=vdt)
    g.refilled = flag
    return g


class _BlockBucket:
    """Static, padded copies of one bucket's inputs: the layer-0 features
    [Cb, D], the seed labels (padding entries -100, which the loss ignores)
    and, per layer, a BCSR block of Rb rows over Cb columns (windows past the
    batch's own hold no tiles) plus, where the backward runs it, its
    transpose.  Padding rows of the features are finite (zeros or an earlier
    batch's rows) and no column index of a block reaches them; padding rows
    of a layer's output have no neighbours and carry zero loss gradient, so
    the padded step computes the batch's loss and gradients."""

    def __init__(self, key, blocks, feat_dtype, feat_dim, needs_t, device):
        rows, c0, fanouts, tc = key[0], key[1], key[2], key[3]
        self.X = torch.zeros((c0, feat_dim), dtype=feat_dtype, device=device)
        self.labels = torch.full((rows[-1],), -100, dtype=torch.int64, device=device)
        self.graphs, self.AT = [], []
        cols = [c0] + list(rows[:-1])
        for l, b in enumerate(blocks):
            R, C, k = rows[l], cols[l], fanouts[l]
            vdt = b.values_condensed.dtype
            W = R // 16
            # a window holds at most 16 k column slots
            g = _bcsr_buffers(R, C, W, W * ((16 * k + tc - 1) // tc), tc, vdt, device, True)
            g.columns_local = True
            g.max_window_slabs = (16 * k + 15) // 16
            g.fanout = k
            at = None
            if needs_t[l]:
                # tiles of A^T: one partial tile per window at most, plus the
                # R k edges in full tiles
                Wt = C // 16
                Tt = Wt + (R * k + tc - 1) // tc
                at = _bcsr_buffers(C, 16 * W, Wt, Tt, tc, vdt, device, True)
                at.max_window_slabs = (Tt * tc + 15) // 16
            self.graphs.append(g)
            self.AT.append(at)

    @staticmethod
    def _copy_bcsr(dst, src) -> None:
        W, T, tc = src.num_windows, src.num_tiles, src.tile_cols
        if W > dst.num_windows or T > dst.num_tiles or src.tile_cols != dst.tile_cols:
            raise ValueError(f"GraphedBlockStep: a block of {W} windows / {T} tiles exceeds its bucket "
                             f"({dst.num_windows} / {dst.num_tiles})")
        dst.window_offset[: W + 1].copy_(src.window_offset)
        dst.window_offset[W + 1:].fill_(T)
        dst.original_col_indices[: T * tc].copy_(src.original_col_indices)
        dst.values_condensed[: T * 16 * tc].copy_(src.values_condensed)

    def fill(self, blocks, feats, labels) -> None:
        """Copies one batch in, on the current stream: every array in one
        copy launch and every padding fill (labels past the batch's, window
        offsets past its windows) in one fill launch when the operands allow
        (core.ops.copy_and_fill), else one torch copy or fill per array."""
        from ..core.ops import TensorKey, copy_and_fill
        pairs = [(g, b) for g, b in zip(self.graphs, blocks)]
        pairs += [(at, b.transpose()) for at, b in zip(self.AT, blocks) if at is not None]
        copies = [(self.X[: feats.shape[0]], feats), (self.labels[: labels.numel()], labels)]
        fills = [(self.labels[labels.numel():], -100)]
        for dst, src in pairs:
            W, T, tc = src.num_windows, src.num_tiles, src.tile_cols
            if W > dst.num_windows or T > dst.num_tiles or src.tile_cols != dst.tile_cols:
                raise ValueError(f"GraphedBlockStep: a block of {W} windows / {T} tiles exceeds its bucket "
                                 f"({dst.num_windows} / {dst.num_tiles})")
            copies += [(dst.window_offset[: W + 1], src.window_offset),
                       (dst.original_col_indices[: T * tc], src.original_col_indices),
                       (dst.values_condensed[: T * 16 * tc], src.values_condensed)]
            fills.append((dst.window_offset[W + 1:], T))
        if not copy_and_fill(copies, fills):
            self.X[: feats.shape[0]].copy_(feats)
            self.labels[: labels.numel()].copy_(labels)
            self.labels[labels.numel():].fill_(-100)
            for dst, src in pairs:
                self._copy_bcsr(dst, src)
        for g, at in zip(self.graphs, self.AT):
            if at is not None:
                # the layer's backward finds the static transpose through the
                # graph's cache, keyed by the arrays' current versions
                arrays = (g.window_offset, g.original_col_indices, g.values_condensed)
                g._cache["T"] = (TensorKey(arrays, (g.num_cols,)), at)


class GraphedBlockStep:
    """The node-wise mini-batch training step (forward over the sampled
    blocks, cross-entropy on the seed rows, backward, clip_grad_norm_(1.0),
    optimizer step; engine.py:86-256 of the reference) captured on a HIP
    graph once per bucket of batch shapes and replayed.

    A batch's shapes (each block's destination count and the input count)
    round up to a bucket (``bucket_rows``).  Its blocks, their transposes,
    the input features and the seed labels are copied into the bucket's
    static buffers (about 20 small device copies), then the bucket's graph
    replays the step: the host issues a few dozen calls per batch instead of
    several hundred kernel launches.

    The first batch of a new bucket runs ``warmup`` eager steps on the
    static buffers, then the capture; parameters, buffers and optimizer
    state are put back as they were before the warm-up (state that the
    warm-up created is zeroed: Adam's and AdamW's initial state), so every
    batch trains exactly once, as in the eager loop.  Dropout draws a new
    mask on every replay.  Needs an optimizer that steps on the device
    (capturable=True) and a model whose hidden layers normalise per row
    (LayerNorm).  Returns (loss, correct) as device tensors that the next
    replay of the same bucket overwrites.  After a capture, a parameter's
    ``.grad`` is that capture's gradient buffer; other buckets' replays write
    their own."""

    def __init__(self, model, optimizer, device, autocast_dtype=None, warmup: int = 1,
                 max_buckets: int = 32):
        if not optimizer.defaults.get("capturable", False):
            raise ValueError("GraphedBlockStep needs an optimizer that steps on the device: build it "
                             "with capturable=True (e.g. torch.optim.Adam(params, capturable=True))")
        for m in model.modules():
            if isinstance(m, torch.nn.modules.batchnorm._BatchNorm):
                raise ValueError("GraphedBlockStep: batch normalisation would see the padding rows")
        self.model, self.opt, self.device = model, optimizer, device
        self.dtype = autocast_dtype
        self.warmup = max(1, int(warmup))
        self.max_buckets = int(max_buckets)
        self.buckets = {}
        self.captures = 0

    def key_of(self, blocks, feats):
        rows = tuple(bucket_rows(b.num_rows) for b in blocks)
        return (rows, bucket_rows(feats.shape[0]), tuple(int(b.fanout) for b in blocks),
                blocks[0].tile_cols, feats.dtype, blocks[0].values_condensed.dtype)

    def _eager(self, bk):
        from .engine import loss_and_metrics_rows
        self.model.train()
        self.opt.zero_grad()
        if self.dtype is None:
            logits = self.model(bk.graphs, bk.X)
        else:
            with torch.autocast("cuda", dtype=self.dtype):
                logits = self.model(bk.graphs, bk.X)
        loss, correct, _ = loss_and_metrics_rows(logits, None, bk.labels)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(self.model.parameters(), max_norm=1.0)
        self.opt.step()
        return loss.detach(), correct

    def _state_tensors(self):
        out = list(self.model.parameters()) + list(self.model.buffers())
        for st in self.opt.state.values():
            out += [v for v in st.values() if torch.is_tensor(v)]
        return out

    def _capture(self, key, blocks, feats, labels):
        from .engine import _transpose_needs
        needs_t = _transpose_needs(self.model, feats)
        bk = _BlockBucket(key, blocks, feats.dtype, feats.shape[1], needs_t, self.device)
        bk.fill(blocks, feats, labels)
        saved = {id(t): (t, t.detach().clone()) for t in self._state_tensors()}
        cur = torch.cuda.current_stream(self.device)
        side = torch.cuda.Stream(self.device)
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            for _ in range(self.warmup):
                self._eager(bk)
        cur.wait_stream(side)
        bk.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(bk.graph, capture_error_mode="thread_local"):
            bk.loss, bk.correct = self._eager(bk)
        # the capture recorded the step without running it; undo the warm-up
        with torch.no_grad():
            for t in self._state_tensors():
                ent = saved.get(id(t))
                if ent is not None and ent[0] is t:
                    t.copy_(ent[1])
                else:
                    t.zero_()
        self.captures += 1
        return bk

    def __call__(self, blocks, feats, labels):
        """One training step on one batch: blocks (destination-first, the
        node-wise sampler's), feats = the input rows' features, labels =
        the seeds' labels (the first rows of the output)."""
        if labels.numel() != blocks[-1].num_rows:
            raise ValueError("GraphedBlockStep: one label per seed (the last block's rows)")
        key = self.key_of(blocks, feats)
        bk = self.buckets.get(key)
        if bk is None:
            if len(self.buckets) >= self.max_buckets:
                self.buckets.pop(next(iter(self.buckets)))
            bk = self._capture(key, blocks, feats, labels)
            self.buckets[key] = bk
        else:
            bk.fill(blocks, feats, labels)
        bk.graph.replay()
        return bk.loss, bk.correct
