"""grws_spmm_noalloc (the SpMM whose split-window partials live in the
library's own device array) against grws_spmm_residual with a caller
workspace, through the C ABI.  Two calls in a row, the second on a smaller
graph and width, so a stale partial left by the first call would show; the
results must be bit-identical (same kernels, same summation order) and within
the north_star bound of the float64 oracle."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from graph_rws_amd import core, synth
from graph_rws_amd.core import _lib as L
from graph_rws_amd.data import BCSRGraph

pytestmark = pytest.mark.gpu

SCRATCH = 16 << 20  # GRWS_SPMM_NOALLOC_SCRATCH_BYTES


def _graph(n, nnz, seed, dev):
    g = synth.chung_lu(n, nnz, 2.1, seed=seed)
    win, cols, vals = core.csr_to_bcsr_cpu(g.num_nodes, g.row_ptr, g.col_idx, g.values, 16, 16)
    return BCSRGraph(g.num_nodes, g.nnz, 16, 16, win, cols, vals, device=dev, num_cols=g.num_nodes,
                     values_dtype=torch.float16)


def _views(G, plan):
    view = L.BcsrView(L.ptr(G.window_offset), L.ptr(G.original_col_indices), L.ptr(G.values_condensed),
                      G.num_windows, G.num_tiles, 16, 16, L.GRWS_F16, 0)
    return view, plan.view()


def _pair(G, plan, X, R):
    """(workspace entry point, allocation-free entry point) results."""
    lib = L.load()
    dev = X.device
    view, pv = _views(G, plan)
    N = X.shape[1]
    rows = 16 * G.num_windows
    y_ws = torch.full((rows, N), float("nan"), dtype=X.dtype, device=dev)
    y_na = torch.full((rows, N), float("nan"), dtype=X.dtype, device=dev)
    wsb = int(lib.grws_spmm_workspace_bytes(ctypes.byref(pv), N))
    assert 0 < wsb <= SCRATCH
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    s = L.stream_of(dev)
    L.call("grws_spmm_residual", ctypes.byref(view), None, ctypes.byref(pv), L.ptr(X), L.GRWS_F16,
           X.shape[0], X.stride(0), N, L.ptr(R), R.stride(0), R.shape[0], L.ptr(y_ws), L.GRWS_F16,
           y_ws.stride(0), L.ptr(ws), wsb, s)
    L.call("grws_spmm_noalloc", ctypes.byref(view), None, ctypes.byref(pv), L.ptr(X), L.GRWS_F16,
           X.shape[0], X.stride(0), N, L.ptr(R), R.stride(0), R.shape[0], L.ptr(y_na), L.GRWS_F16,
           y_na.stride(0), s)
    torch.cuda.synchronize()
    return y_ws, y_na


def _oracle_check(G, X, R, Y):
    vq = G.values_condensed.double().cpu().numpy()
    Yr, Ya = oracle.bcsr_spmm(G.window_offset.cpu().numpy(), G.original_col_indices.cpu().numpy(),
                              vq, 16, 16, X.double().cpu().numpy())
    Rd = R.double().cpu().numpy()
    Yr[:Rd.shape[0]] += Rd
    Ya[:Rd.shape[0]] += np.abs(Rd)
    err = np.abs(Y.double().cpu().numpy() - Yr)
    assert (err <= 1e-2 * Ya + 1e-3 * np.abs(Yr)).all(), f"max err {err.max():.3e}"


def test_noalloc_matches_workspace_entry_point(cuda_device):
    print("case noalloc: chung_lu 3000 N=128 (4 slabs) then 1500 N=48 (8 slabs)", flush=True)
    # (nodes, edges, seed, N, slabs per item): 10.6 MB, then 1.2 MB of partials
    cases = [(3000, 40000, 11, 128, 4), (1500, 15000, 12, 48, 8)]
    for n, nnz, seed, N, slabs in cases:
        G = _graph(n, nnz, seed, cuda_device)
        plan = core.build_spmm_plan(G.window_offset, G.num_tiles, 16, slabs)
        assert plan.num_split > 0, "the case must split windows so the scratch is used"
        X = synth.features(n, N, seed=seed, device=cuda_device).half()
        R = synth.features(n // 2, N, seed=seed + 1, device=cuda_device).half()
        y_ws, y_na = _pair(G, plan, X, R)
        assert torch.equal(y_ws.view(torch.int16), y_na.view(torch.int16)), f"n={n} N={N}: results differ"
        _oracle_check(G, X, R, y_na)


def test_noalloc_rejects_plans_past_the_scratch(cuda_device):
    """A plan whose partials exceed the scratch is refused on the host."""
    print("case noalloc: capacity refusal", flush=True)
    lib = L.load()
    G = _graph(3000, 40000, 11, cuda_device)
    plan = core.build_spmm_plan(G.window_offset, G.num_tiles, 16, 1)
    view, pv = _views(G, plan)
    N = 1024
    need = int(lib.grws_spmm_workspace_bytes(ctypes.byref(pv), N))
    assert need > SCRATCH
    X = torch.zeros((3000, N), dtype=torch.float16, device=cuda_device)
    Y = torch.empty((16 * G.num_windows, N), dtype=torch.float16, device=cuda_device)
    st = lib.grws_spmm_noalloc(ctypes.byref(view), None, ctypes.byref(pv), L.ptr(X), L.GRWS_F16, 3000, N, N,
                               None, 0, 0, L.ptr(Y), L.GRWS_F16, N, L.stream_of(cuda_device))
    assert st == L.GRWS_E_CAPACITY
    assert b"scratch" in lib.grws_last_error()


def test_noalloc_refuses_a_stream_of_another_device(cuda_device):
    """The scratch array belongs to the current device: a stream of another
    device is refused with GRWS_E_INVALID before any kernel is launched.
    Needs two GPUs (a one-GPU box has no stream of another device)."""
    if torch.cuda.device_count() < 2:
        pytest.skip("needs a second GPU for a stream of another device")
    print("case noalloc stream of another device", flush=True)
    G = _graph(3000, 60000, 5, cuda_device)
    plan = core.build_spmm_plan(G.window_offset, G.num_tiles, 16, 2)
    X = torch.randn(G.num_cols, 64, device=cuda_device).half()
    R = torch.zeros(0, 64, device=cuda_device).half()
    Y = torch.empty(16 * G.num_windows, 64, device=cuda_device).half()
    view, pv = _views(G, plan)
    other = torch.cuda.Stream(device=torch.device("cuda", 1))
    st = L.load().grws_spmm_noalloc(ctypes.byref(view), None, ctypes.byref(pv), L.ptr(X), L.GRWS_F16,
                                    X.shape[0], X.stride(0), 64, L.ptr(R), R.stride(0), 0, L.ptr(Y),
                                    L.GRWS_F16, Y.stride(0), ctypes.c_void_p(other.cuda_stream))
    assert st == L.GRWS_E_INVALID
    assert b"belongs to device" in L.load().grws_last_error()
