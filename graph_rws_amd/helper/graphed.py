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
        with torch.cuda.graph(self.graph):
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
