"""WindowWiseDataLoader (data/data_loader.py:39-115 of the reference):
training nodes grouped by 16-row window; each epoch shuffles the windows and
yields whole windows until a batch holds at least batch_size nodes."""
from __future__ import annotations

import numpy as np
import torch


class WindowWiseDataLoader:
    def __init__(self, train_idx: torch.Tensor, batch_size: int, tile_rows: int = 16,
                 drop_last: bool = False, generator: torch.Generator = None):
        self.batch_size = int(batch_size)
        self.drop_last = drop_last
        self.device = train_idx.device
        self.generator = generator
        idx = train_idx.cpu()
        wids = idx.div(tile_rows, rounding_mode="floor")
        order = torch.argsort(wids, stable=True)
        self.sorted_train_idx = idx[order]
        _, counts = torch.unique_consecutive(wids[order], return_counts=True)
        starts = torch.cumsum(counts, 0) - counts
        self.num_windows = int(counts.numel())
        self._starts = starts.numpy().astype(np.int64)
        self._counts = counts.numpy().astype(np.int64)
        self._sorted_np = self.sorted_train_idx.numpy()
        self._window_info = None

    @property
    def window_info(self):
        """[(start, count)] per window in sorted_train_idx (data_loader.py:74-80),
        built on first use: the batches come from the arrays above, and a
        list of one tuple per window (~40k for a c5 epoch) cost milliseconds
        and garbage-collector passes at every epoch's start."""
        if self._window_info is None:
            self._window_info = list(zip(self._starts.tolist(), self._counts.tolist()))
        return self._window_info

    def __iter__(self):
        """Same batches as walking the shuffled windows one by one
        (data_loader.py:87-110), found with one search per batch: a batch
        ends at the first window where its node count reaches batch_size,
        and its nodes are gathered with one vector op (c5 batches span ~1,000
        windows of one node each)."""
        perm = torch.randperm(self.num_windows, generator=self.generator).numpy()
        counts = self._counts[perm]
        starts = self._starts[perm]
        csum = np.cumsum(counts)
        total = int(csum[-1]) if csum.size else 0
        i, base = 0, 0
        while i < self.num_windows:
            if total - base >= self.batch_size:
                j = max(i, int(np.searchsorted(csum, base + self.batch_size, side="left")))
            elif self.drop_last:
                return
            else:
                j = self.num_windows - 1
            c = counts[i:j + 1]
            first = np.cumsum(c) - c
            pos = np.repeat(starts[i:j + 1] - first, c) + np.arange(int(c.sum()))
            yield torch.from_numpy(self._sorted_np[pos]).to(self.device)
            base = int(csum[j])
            i = j + 1

    def __len__(self):
        """Estimated batch count (data_loader.py:112-115)."""
        return (len(self.sorted_train_idx) + self.batch_size - 1) // self.batch_size
