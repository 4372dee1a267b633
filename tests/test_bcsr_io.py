"""On-disk BCSR cache (graph_rws_amd/data/bcsr_io.py, the reference's
data/data_loader.py:282-406): the golden fixture in the reference layout,
round trips through save/load (read and memory-mapped), the reference's
failure rules, and (GPU) streaming into HBM through pinned chunks."""
import os
import sys

import numpy as np
import pytest
import torch

from graph_rws_amd import core, synth
from graph_rws_amd.data import (BCSRGraph, bcsr_bin_paths, estimate_bcsr_bytes, load_bcsr_bins,
                                make_bcsr_stub, save_bcsr_bins)

GOLD = os.path.join(os.path.dirname(__file__), "golden", "bcsr_io", "g.pt")
sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
import make_bcsr_io_fixture as fx  # noqa: E402


@pytest.mark.parametrize("mmap", [False, True])
def test_golden_fixture_loads(mmap):
    g, used = load_bcsr_bins(GOLD, force_mmap=mmap)
    assert used == mmap
    assert (g.num_nodes, g.num_edges, g.num_rows, g.num_cols, g.tile_rows, g.tile_cols, g.num_windows) == \
        (20, 12, 20, 20, 16, 8, 2)
    assert g.window_offset.tolist() == fx.offsets
    assert g.original_col_indices.tolist() == fx.cols
    np.testing.assert_array_equal(g.values_condensed.numpy(), np.array(fx.vals, np.float32))
    # the file is opened copy-on-write: writing through the tensor leaves it intact
    if mmap:
        g.values_condensed[0] = 123.0
        g2, _ = load_bcsr_bins(GOLD, force_mmap=True)
        assert float(g2.values_condensed[0]) == fx.vals[0]


def _graph(tc=16):
    s = synth.random_graph(300, 6.0, seed=4)
    win, cols, vals = core.csr_to_bcsr_cpu(s.num_nodes, s.row_ptr, s.col_idx, s.values, 16, tc)
    return BCSRGraph(s.num_nodes, s.nnz, 16, tc, win, cols, vals, device=torch.device("cpu"),
                     num_cols=s.num_nodes)


@pytest.mark.parametrize("tc", [8, 16])
def test_round_trip(tmp_path, tc):
    G = _graph(tc)
    path = str(tmp_path / "cache.pt")
    assert save_bcsr_bins(G, path)
    for p in bcsr_bin_paths(path):
        assert os.path.exists(p)
    # raw layout: file sizes are exactly the arrays
    _, off_p, col_p, val_p = bcsr_bin_paths(path)
    assert os.path.getsize(off_p) == 8 * G.window_offset.numel()
    assert os.path.getsize(col_p) == 4 * G.original_col_indices.numel()
    assert os.path.getsize(val_p) == 4 * G.values_condensed.numel()
    for mmap in (False, True):
        H, used = load_bcsr_bins(path, force_mmap=mmap)
        assert used == mmap
        assert torch.equal(H.window_offset, G.window_offset)
        assert torch.equal(H.original_col_indices, G.original_col_indices)
        assert torch.equal(H.values_condensed, G.values_condensed)
        assert (H.num_nodes, H.num_edges, H.num_rows, H.num_cols, H.num_windows) == \
            (G.num_nodes, G.num_edges, G.num_rows, G.num_cols, G.num_windows)
    H16, _ = load_bcsr_bins(path, values_dtype=torch.float16)
    assert H16.values_condensed.dtype == torch.float16
    assert torch.equal(H16.values_condensed, G.values_condensed.half())


def test_low_precision_graph_saved_as_float32(tmp_path):
    G = _graph()
    G16 = BCSRGraph(G.num_nodes, G.num_edges, 16, 16, G.window_offset, G.original_col_indices,
                    G.values_condensed, device=torch.device("cpu"), values_dtype=torch.bfloat16)
    path = str(tmp_path / "c.pt")
    assert save_bcsr_bins(G16, path)
    H, _ = load_bcsr_bins(path)
    assert H.values_condensed.dtype == torch.float32
    assert torch.equal(H.values_condensed, G16.values_condensed.float())


def test_missing_and_mismatched_files(tmp_path):
    G = _graph()
    path = str(tmp_path / "m.pt")
    assert load_bcsr_bins(path) == (None, False)
    assert save_bcsr_bins(G, path)
    _, _, col_p, _ = bcsr_bin_paths(path)
    with open(col_p, "ab") as f:
        f.write(b"\0\0\0\0")
    assert load_bcsr_bins(path) == (None, False)
    os.remove(col_p)
    assert load_bcsr_bins(path) == (None, False)


def test_estimate_and_stub():
    G = _graph()
    assert estimate_bcsr_bytes(G) == 8 * G.window_offset.numel() + 4 * G.original_col_indices.numel() \
        + 4 * G.values_condensed.numel()
    s = make_bcsr_stub(G)
    assert s.is_stub and s.num_windows == G.num_windows and s.num_nodes == G.num_nodes
    assert s.window_offset.numel() == 1


@pytest.mark.gpu
@pytest.mark.parametrize("vdt", [torch.float32, torch.float16, torch.bfloat16])
def test_stream_into_hbm(tmp_path, cuda_device, vdt):
    """Device load through pinned chunks (a 4 KiB chunk forces many) equals
    the host load, values converted on the device."""
    print(f"case bcsr_io device {vdt}", flush=True)
    G = _graph()
    path = str(tmp_path / "d.pt")
    assert save_bcsr_bins(G, path)
    H, _ = load_bcsr_bins(path, device=cuda_device, values_dtype=vdt, chunk_bytes=4096)
    torch.cuda.synchronize()
    assert H.window_offset.is_cuda and H.values_condensed.dtype == vdt
    assert torch.equal(H.window_offset.cpu(), G.window_offset)
    assert torch.equal(H.original_col_indices.cpu(), G.original_col_indices)
    assert torch.equal(H.values_condensed.cpu(), G.values_condensed.to(vdt))
    # and the loaded graph multiplies like the original
    X = torch.randn(G.num_cols, 32, device=cuda_device)
    Gd = BCSRGraph(G.num_nodes, G.num_edges, 16, 16, G.window_offset, G.original_col_indices,
                   G.values_condensed, device=cuda_device, values_dtype=vdt)
    assert torch.equal(H.spmm(X.to(vdt) if vdt != torch.float32 else X),
                       Gd.spmm(X.to(vdt) if vdt != torch.float32 else X))
