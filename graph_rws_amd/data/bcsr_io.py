"""On-disk BCSR format (data/data_loader.py:282-406 of the reference).

A graph cached at ``<name>.pt`` is stored as four files beside it:

  ``<name>_bcsr_meta.pt``           dict of ints written by ``torch.save``:
                                    num_nodes, num_edges, num_rows, num_cols,
                                    tile_rows, tile_cols, num_windows,
                                    window_offset_len, col_indices_len,
                                    values_len
  ``<name>_bcsr_window_offset.bin`` raw int64, little-endian
  ``<name>_bcsr_col_indices.bin``   raw int32
  ``<name>_bcsr_values.bin``        raw float32

Same names, layout and metadata keys as the reference, so caches written by
either side load in the other.  Loading follows the reference's rule for host
memory (memory-map the files when twice their size exceeds MemAvailable,
data_loader.py:355-357) and adds a device path: with a CUDA ``device`` the
arrays are streamed from the (memory-mapped) files straight into HBM through
two pinned staging buffers, so a multi-GB graph never sits whole in host
memory, and the values can be converted to float16 / bfloat16 on the device
chunk by chunk.  The metadata is read with ``torch.load(weights_only=True)``
(plain ints only; nothing in the file is executed).
"""
from __future__ import annotations

import os
from typing import Optional, Tuple

import numpy as np
import torch

from .bcsr import BCSRGraph

_ITEM = {"window_offset": (np.int64, 8), "col_indices": (np.int32, 4), "values": (np.float32, 4)}

# bytes per staging buffer for host -> device streaming
STREAM_CHUNK_BYTES = 64 << 20


def bcsr_bin_paths(cache_path: str) -> Tuple[str, str, str, str]:
    """(meta, window_offset, col_indices, values) paths for a cache path
    (data_loader.py:282-287)."""
    return (cache_path.replace(".pt", "_bcsr_meta.pt"),
            cache_path.replace(".pt", "_bcsr_window_offset.bin"),
            cache_path.replace(".pt", "_bcsr_col_indices.bin"),
            cache_path.replace(".pt", "_bcsr_values.bin"))


def estimate_bcsr_bytes(bcsr: BCSRGraph) -> int:
    """Bytes of the three BCSR arrays as held (data_loader.py:290-298)."""
    total = 0
    for name in ("window_offset", "original_col_indices", "values_condensed"):
        t = getattr(bcsr, name, None)
        if t is not None:
            total += t.numel() * t.element_size()
    return int(total)


def make_bcsr_stub(bcsr: BCSRGraph) -> BCSRGraph:
    """A CPU placeholder with the graph's sizes and one-element arrays
    (data_loader.py:301-320)."""
    dev = torch.device("cpu")
    stub = BCSRGraph(num_nodes=int(bcsr.num_nodes), num_edges=0, tile_rows=int(bcsr.tile_rows),
                     tile_cols=int(bcsr.tile_cols),
                     window_offset=torch.zeros(1, dtype=torch.int64),
                     original_col_indices=torch.zeros(1, dtype=torch.int32),
                     values_condensed=torch.zeros(1, dtype=torch.float32), device=dev,
                     num_rows=int(bcsr.num_rows), num_cols=int(bcsr.num_cols))
    stub.num_windows = int(getattr(bcsr, "num_windows", 0))
    stub.is_stub = True
    return stub


def save_bcsr_bins(bcsr: BCSRGraph, cache_path: str) -> bool:
    """Writes the four files (data_loader.py:323-350).  Values are stored as
    float32 whatever dtype the graph holds.  Returns False (and prints why)
    if writing fails, as the reference does."""
    meta_path, off_path, col_path, val_path = bcsr_bin_paths(cache_path)
    try:
        off = bcsr.window_offset.detach().to("cpu", torch.int64).contiguous()
        col = bcsr.original_col_indices.detach().to("cpu", torch.int32).contiguous()
        val = bcsr.values_condensed.detach().to("cpu", torch.float32).contiguous()
        off.numpy().astype("<i8", copy=False).tofile(off_path)
        col.numpy().astype("<i4", copy=False).tofile(col_path)
        val.numpy().astype("<f4", copy=False).tofile(val_path)
        meta = {
            "num_nodes": int(bcsr.num_nodes), "num_edges": int(bcsr.num_edges),
            "num_rows": int(bcsr.num_rows), "num_cols": int(bcsr.num_cols),
            "tile_rows": int(bcsr.tile_rows), "tile_cols": int(bcsr.tile_cols),
            "num_windows": int(getattr(bcsr, "num_windows", 0)),
            "window_offset_len": int(off.numel()), "col_indices_len": int(col.numel()),
            "values_len": int(val.numel()),
        }
        torch.save(meta, meta_path)
        return True
    except Exception as e:  # the reference reports and carries on
        print(f"[Data] Failed to save BCSR bins: {e}")
        return False


def mem_available_bytes() -> int:
    """MemAvailable from /proc/meminfo, or -1 (data_loader.py:270-279)."""
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemAvailable:"):
                    return int(line.split()[1]) * 1024
    except OSError:
        return -1
    return -1


def _read_meta(meta_path: str) -> dict:
    meta = torch.load(meta_path, weights_only=True)
    if not isinstance(meta, dict):
        raise ValueError(f"{meta_path}: metadata is not a dict")
    return {k: int(v) for k, v in meta.items()}


def _stream_to_device(arr: np.ndarray, device: torch.device, out_dtype: torch.dtype,
                      chunk_bytes: int) -> torch.Tensor:
    """Copies a host array (possibly memory-mapped) into a new device tensor
    of out_dtype in chunks through two pinned buffers: chunk i+1 is read
    from the file while chunk i is in flight."""
    src_dt = torch.from_numpy(arr[:0]).dtype
    n = int(arr.shape[0])
    out = torch.empty(n, dtype=out_dtype, device=device)
    if n == 0:
        return out
    copy_stream = torch.cuda.Stream(device)
    out.record_stream(copy_stream)
    per = max(1, chunk_bytes // arr.itemsize)
    stage = [torch.empty(min(per, n), dtype=src_dt, pin_memory=True) for _ in range(2)]
    done = [None, None]
    with torch.cuda.stream(copy_stream):
        for k, lo in enumerate(range(0, n, per)):
            hi = min(n, lo + per)
            buf = stage[k % 2]
            if done[k % 2] is not None:
                done[k % 2].synchronize()  # the previous copy out of this buffer ended
            buf[: hi - lo].numpy()[:] = arr[lo:hi]
            if out_dtype == src_dt:
                out[lo:hi].copy_(buf[: hi - lo], non_blocking=True)
            else:
                tmp = buf[: hi - lo].to(device, non_blocking=True)
                out[lo:hi].copy_(tmp)
            ev = torch.cuda.Event()
            ev.record(copy_stream)
            done[k % 2] = ev
    torch.cuda.current_stream(device).wait_stream(copy_stream)
    return out


def load_bcsr_bins(cache_path: str, device: Optional[torch.device] = None,
                   values_dtype: torch.dtype = torch.float32, force_mmap: Optional[bool] = None,
                   chunk_bytes: int = STREAM_CHUNK_BYTES) -> Tuple[Optional[BCSRGraph], bool]:
    """Loads a cached graph (data_loader.py:353-406).  Returns
    (graph, used_memmap), or (None, False) when a file is missing or the
    metadata and file sizes disagree, as the reference does.

    device None / CPU: CPU tensors over the files' data (memory-mapped when
    ``force_mmap`` or twice the total exceeds MemAvailable).  A CUDA device:
    the arrays are streamed into HBM (``values_dtype`` applied on the
    device)."""
    meta_path, off_path, col_path, val_path = bcsr_bin_paths(cache_path)
    if not all(os.path.exists(p) for p in (meta_path, off_path, col_path, val_path)):
        return None, False
    meta = _read_meta(meta_path)
    lens = {"window_offset": meta.get("window_offset_len", 0), "col_indices": meta.get("col_indices_len", 0),
            "values": meta.get("values_len", 0)}
    if min(lens.values()) <= 0:
        return None, False
    paths = {"window_offset": off_path, "col_indices": col_path, "values": val_path}
    for k, p in paths.items():
        if os.path.getsize(p) != lens[k] * _ITEM[k][1]:
            print("[Data] BCSR binary shape mismatch, ignoring bins.")
            return None, False
    total = sum(lens[k] * _ITEM[k][1] for k in lens)
    if force_mmap is None:
        avail = mem_available_bytes()
        use_mmap = avail > 0 and total * 2 > avail
    else:
        use_mmap = bool(force_mmap)
    dev = torch.device(device) if device is not None else torch.device("cpu")
    if dev.type == "cuda":
        use_mmap = True  # the device path reads the files through the page cache
    arrs = {}
    for k, p in paths.items():
        dt = np.dtype(_ITEM[k][0]).newbyteorder("<")
        if use_mmap:
            # copy-on-write mapping: writable views for torch, the file is never modified
            arrs[k] = np.memmap(p, dtype=dt, mode="c", shape=(lens[k],))
        else:
            arrs[k] = np.fromfile(p, dtype=dt)
    if dev.type == "cuda":
        off = _stream_to_device(arrs["window_offset"], dev, torch.int64, chunk_bytes)
        col = _stream_to_device(arrs["col_indices"], dev, torch.int32, chunk_bytes)
        val = _stream_to_device(arrs["values"], dev, values_dtype, chunk_bytes)
    else:
        off = torch.from_numpy(np.asarray(arrs["window_offset"]).view(np.int64))
        col = torch.from_numpy(np.asarray(arrs["col_indices"]).view(np.int32))
        val = torch.from_numpy(np.asarray(arrs["values"]).view(np.float32))
        if values_dtype != torch.float32:
            val = val.to(values_dtype)
    g = BCSRGraph(num_nodes=meta["num_nodes"], num_edges=meta["num_edges"], tile_rows=meta["tile_rows"],
                  tile_cols=meta["tile_cols"], window_offset=off, original_col_indices=col,
                  values_condensed=val, device=dev, num_rows=meta["num_rows"], num_cols=meta["num_cols"],
                  values_dtype=values_dtype)
    g.num_windows = int(meta.get("num_windows", g.num_windows))
    return g, use_mmap
