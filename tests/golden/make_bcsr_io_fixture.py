"""Writes tests/golden/bcsr_io/g_*: a tiny BCSR cache in the reference's
on-disk layout (data/data_loader.py:323-350): raw little-endian int64 window
offsets, int32 column indices, float32 values, and a torch.save'd dict of
ints.  The bytes are packed with `struct` here (not numpy), so the fixture
pins the layout independently of graph_rws_amd.data.bcsr_io.

Graph: 20 nodes, tile 16x8, 2 windows; window 0 has columns {1, 5, 19}
(one tile, -1 padded), window 1 has columns {0, 2, 3, 4, 6, 7, 8, 9, 12}
(two tiles).  Values: tile t, row r, column c holds t + r/16 + c/256 where
the column slot is used, 0 elsewhere."""
import os
import struct

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "bcsr_io", "g.pt")

offsets = [0, 1, 3]
cols = [1, 5, 19, -1, -1, -1, -1, -1,
        0, 2, 3, 4, 6, 7, 8, 9,
        12, -1, -1, -1, -1, -1, -1, -1]
vals = []
for t in range(3):
    for r in range(16):
        for c in range(8):
            used = cols[t * 8 + c] >= 0
            vals.append(t + r / 16 + c / 256 if used else 0.0)

if __name__ == "__main__":
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    base = OUT.replace(".pt", "")
    with open(base + "_bcsr_window_offset.bin", "wb") as f:
        f.write(struct.pack("<%dq" % len(offsets), *offsets))
    with open(base + "_bcsr_col_indices.bin", "wb") as f:
        f.write(struct.pack("<%di" % len(cols), *cols))
    with open(base + "_bcsr_values.bin", "wb") as f:
        f.write(struct.pack("<%df" % len(vals), *vals))
    meta = {"num_nodes": 20, "num_edges": 12, "num_rows": 20, "num_cols": 20, "tile_rows": 16,
            "tile_cols": 8, "num_windows": 2, "window_offset_len": len(offsets),
            "col_indices_len": len(cols), "values_len": len(vals)}
    torch.save(meta, base + "_bcsr_meta.pt")
    print("wrote", base + "_bcsr_*")
