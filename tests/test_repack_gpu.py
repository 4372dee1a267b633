"""Halo repack on the device (csrc/repack.hip via BCSRSampler.repack_subgraph)
against oracle.repack_subgraph (sampler/sampler.py:420-690): integer arrays
bit-exact, values exact (they are copied or zeroed, never computed)."""
import numpy as np
import pytest
import torch

import oracle
from graph_rws_amd import synth
from graph_rws_amd.core._lib import GrwsError
from graph_rws_amd.data import BCSRGraph
from graph_rws_amd.sampler import BCSRSampler

pytestmark = pytest.mark.gpu


def _graph(dev, n, deg, tc, vdt, seed, kind="powerlaw"):
    if kind == "powerlaw":
        s = synth.chung_lu(n, n * deg, 2.1, seed=seed)
    else:
        s = synth.random_graph(n, float(deg), seed=seed)
    return BCSRGraph.from_csr(s.row_ptr, s.col_idx, s.values, s.num_nodes, s.num_nodes, tile_cols=tc,
                              device=dev, values_dtype=vdt)


def _check(sub, ref, vdt):
    np.testing.assert_array_equal(sub.window_offset.cpu().numpy(), ref["window_offset"])
    np.testing.assert_array_equal(sub.original_node_ids.cpu().numpy(), ref["input_nodes"])
    assert sub.num_internal_nodes == ref["num_internal"] == sub.num_rows
    assert sub.num_cols == ref["input_nodes"].size
    np.testing.assert_array_equal(sub.original_col_indices.cpu().numpy(), ref["halo_cols"])
    np.testing.assert_array_equal(sub.values_condensed.float().cpu().numpy(),
                                  ref["halo_values"].astype(np.float32))
    inner = sub.inner_graph
    np.testing.assert_array_equal(inner.original_col_indices.cpu().numpy(), ref["inner_cols"])
    np.testing.assert_array_equal(inner.values_condensed.float().cpu().numpy(),
                                  ref["inner_values"].astype(np.float32))
    assert inner.num_cols == ref["num_internal"]
    assert sub.num_edges == ref["halo_nnz"] and inner.num_edges == ref["inner_nnz"]
    assert sub.is_local_input and sub.values_condensed.dtype == vdt


def _ref(G, wids, ratio, perm=None):
    vals = G.values_condensed.float().cpu().numpy()
    return oracle.repack_subgraph(G.window_offset.cpu().numpy(), G.original_col_indices.cpu().numpy(),
                                  vals, G.num_nodes, G.tile_cols, wids, ratio, perm=perm)


def _state_clean(s):
    st = s._repack_state_cache
    return bool((st.node_map == -1).all()) and bool((st.bitmap == 0).all())


@pytest.mark.parametrize("tc,vdt", [(8, torch.float32), (16, torch.float32), (16, torch.float16),
                                    (8, torch.bfloat16)])
def test_repack_all_kept(cuda_device, tc, vdt):
    print(f"case repack all-kept tc={tc} {vdt}", flush=True)
    G = _graph(cuda_device, 5003, 12, tc, vdt, seed=3)  # 5003 nodes: the last window is partial
    s = BCSRSampler([5], tile_cols=tc)
    W = G.num_windows
    wids = torch.tensor([W - 1, 0, 7, 100, 5, W + 3, -2], device=cuda_device)  # unsorted + invalid
    sub = s.repack_subgraph(G, wids, max_external_ratio=1e6)
    torch.cuda.synchronize()
    _check(sub, _ref(G, wids.cpu().numpy(), 1e6), vdt)
    assert sub.original_window_ids.tolist() == [0, 5, 7, 100, W - 1]
    assert _state_clean(s)


@pytest.mark.parametrize("tc", [8, 16])
def test_repack_over_budget_matches_reference_draw(cuda_device, tc):
    """More candidates than the budget: the kept subset is the one the
    reference's torch.randperm call on the device would pick."""
    print(f"case repack over-budget tc={tc}", flush=True)
    G = _graph(cuda_device, 20000, 20, tc, torch.float32, seed=5)
    s = BCSRSampler([5], tile_cols=tc)
    wids = torch.arange(0, G.num_windows, 37, device=cuda_device)
    n_ext = _ref(G, wids.cpu().numpy(), 1e9)["num_external"]
    torch.manual_seed(1234)
    sub = s.repack_subgraph(G, wids, max_external_ratio=0.75)
    torch.manual_seed(1234)
    perm = torch.randperm(n_ext, device=cuda_device).cpu().numpy()
    ref = _ref(G, wids.cpu().numpy(), 0.75, perm=perm)
    assert ref["input_nodes"].size - ref["num_internal"] == int(ref["num_internal"] * 0.75) < n_ext
    _check(sub, ref, torch.float32)
    assert _state_clean(s)
    # an explicit generator gives the same subset as the same draw from it
    g1 = torch.Generator(device=cuda_device).manual_seed(7)
    sub2 = s.repack_subgraph(G, wids, max_external_ratio=0.75, generator=g1)
    g2 = torch.Generator(device=cuda_device).manual_seed(7)
    perm2 = torch.randperm(n_ext, device=cuda_device, generator=g2).cpu().numpy()
    _check(sub2, _ref(G, wids.cpu().numpy(), 0.75, perm=perm2), torch.float32)


def test_repack_nan_values(cuda_device):
    """A NaN left in the halo values sends them through nan_to_num (after
    num_edges is counted), and the inner graph copies the cleaned values."""
    print("case repack nan", flush=True)
    G = _graph(cuda_device, 3000, 10, 16, torch.float32, seed=9)
    v = G.values_condensed
    nz = torch.nonzero(v).view(-1)
    v[nz[::50]] = float("nan")
    v[nz[7::50]] = float("inf")
    s = BCSRSampler([5], tile_cols=16)
    wids = torch.arange(0, G.num_windows, 3, device=cuda_device)
    sub = s.repack_subgraph(G, wids, max_external_ratio=1e6)
    ref = _ref(G, wids.cpu().numpy(), 1e6)
    assert not np.isnan(ref["halo_values"]).any() and np.isfinite(ref["halo_values"]).all()
    _check(sub, ref, torch.float32)


def test_repack_edges_and_errors(cuda_device):
    print("case repack edges", flush=True)
    G = _graph(cuda_device, 1000, 8, 16, torch.float32, seed=2, kind="random")
    s = BCSRSampler([5], tile_cols=16)
    sub = s.repack_subgraph(G, torch.empty(0, dtype=torch.int64, device=cuda_device))
    assert sub.num_windows == 0 and sub.original_node_ids.numel() == 0 and sub.num_rows == 0
    sub = s.repack_subgraph(G, torch.tensor([-5, 10 ** 6], device=cuda_device))  # all filtered
    assert sub.num_windows == 0
    with pytest.raises(ValueError, match="duplicate"):
        s.repack_subgraph(G, torch.tensor([3, 3], device=cuda_device))
    with pytest.raises(ValueError, match="tiles"):
        BCSRSampler([5], tile_cols=8).repack_subgraph(G, torch.tensor([1], device=cuda_device))
    assert _state_clean(s)
    # int32 ids are accepted and kept in their dtype
    sub = s.repack_subgraph(G, torch.tensor([4, 2], dtype=torch.int32, device=cuda_device), 1e6)
    _check(sub, _ref(G, np.array([4, 2]), 1e6), torch.float32)
    assert sub.original_window_ids.dtype == torch.int32
    stub = s.repack_subgraph(G, torch.tensor([4, 2], device=cuda_device), dry_run=True)
    assert stub.num_internal_nodes == 32 and stub.total_tiles == int(sub.window_offset[-1])
    assert stub.values_condensed is None


def test_repack_abi_rejects_bad_ids(cuda_device):
    """Unsorted or out-of-range ids passed straight to the C ABI are errors,
    and the state is left clean."""
    from graph_rws_amd.core.ops import SampleState, repack
    G = _graph(cuda_device, 500, 6, 16, torch.float32, seed=4, kind="random")
    st = SampleState(G.num_nodes, cuda_device)
    for bad in ([3, 1], [0, G.num_windows], [2, 2]):
        with pytest.raises(GrwsError, match="window"):
            repack(G.window_offset, G.original_col_indices, G.values_condensed, 16, G.num_nodes,
                   torch.tensor(bad, device=cuda_device), 5.0, st)
        assert bool((st.node_map == -1).all()) and bool((st.bitmap == 0).all())


def test_repacked_graph_multiplies(cuda_device):
    """SpMM over the halo graph with the gathered input features equals the
    original graph's rows of A X restricted to the kept columns (all kept)."""
    G = _graph(cuda_device, 4000, 10, 16, torch.float32, seed=8)
    s = BCSRSampler([5], tile_cols=16)
    wids = torch.arange(3, G.num_windows, 11, device=cuda_device)
    sub = s.repack_subgraph(G, wids, max_external_ratio=1e6)
    X = torch.randn(G.num_nodes, 40, device=cuda_device)
    Y = sub.spmm(X[sub.original_node_ids].contiguous())
    full = G.spmm(X)
    rows = (wids.view(-1, 1) * 16 + torch.arange(16, device=cuda_device)).view(-1)
    ok = rows < G.num_nodes
    torch.testing.assert_close(Y[ok], full[rows[ok]], rtol=1e-5, atol=1e-5)
