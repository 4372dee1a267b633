"""WindowWiseDataLoader (data/data_loader.py:39-115 of the reference):
training nodes grouped by 16-row window; each epoch shuffles the windows and
yields whole windows until a batch holds at least batch_size nodes."""
from __future__ import annotations

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
        self.window_info = list(zip(starts.tolist(), counts.tolist()))
        self.num_windows = len(self.window_info)

    def __iter__(self):
        perm = torch.randperm(self.num_windows, generator=self.generator)
        batch, n = [], 0
        for w in perm.tolist():
            s, c = self.window_info[w]
            batch.append(self.sorted_train_idx[s:s + c])
            n += c
            if n >= self.batch_size:
                yield torch.cat(batch).to(self.device)
                batch, n = [], 0
        if not self.drop_last and batch:
            yield torch.cat(batch).to(self.device)

    def __len__(self):
        """Estimated batch count (data_loader.py:112-115)."""
        return (len(self.sorted_train_idx) + self.batch_size - 1) // self.batch_size
