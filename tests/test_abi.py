"""C-ABI library: loads without a GPU, exports every symbol include/grws.h
declares, and its host-side entry points (sizing, validation, host
converter) behave.  No device compute here.  CPU only."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

import oracle
from graph_rws_amd.core import _lib as L
from graph_rws_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    inc = os.path.join(ROOT, "include")
    for f in os.listdir(inc):
        if not f.endswith(".h"):
            continue
        text = open(os.path.join(inc, f)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(grws_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_library_loads_and_exports_header_symbols():
    lib = L.load()
    declared = _declared_functions()
    assert "grws_spmm" in declared
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    # every prototype the Python binding declares is in the header too
    assert set(L.exported_symbols()) <= set(declared)
    assert lib.grws_abi_version() == 1


def test_plan_capacity_and_errors():
    lib = L.load()
    mi, ms = ctypes.c_int64(), ctypes.c_int64()
    assert lib.grws_spmm_plan_capacity(10, 100, 16, 8, ctypes.byref(mi), ctypes.byref(ms)) == 0
    # 100 tiles of 16 cols = 100 slabs; <= W + slabs/S + 1 items
    assert mi.value >= 10 + 100 // 8 and ms.value <= 10
    st = lib.grws_spmm_plan_capacity(10, 100, 7, 8, ctypes.byref(mi), ctypes.byref(ms))
    assert st == -1
    assert b"tile_cols" in lib.grws_last_error()


def test_spmm_rejects_bad_arguments_without_launching():
    lib = L.load()
    st = lib.grws_spmm(None, None, None, 0, 0, 0, 0, None, 0, 0, None, 0, None)
    assert st == -1 and b"null graph" in lib.grws_last_error()
    view = L.BcsrView(None, None, None, 4, 0, 16, 12, 0, 0)
    st = lib.grws_spmm(ctypes.byref(view), None, None, 0, 0, 0, 8, None, 0, 8, None, 0, None)
    assert st == -1 and b"tile_cols" in lib.grws_last_error()
    view = L.BcsrView(None, None, None, 4, 0, 16, 16, 0, 0)
    st = lib.grws_spmm(ctypes.byref(view), None, None, 1, 0, 0, 8, None, 2, 8, None, 0, None)
    assert st == -2  # y dtype != x dtype


@pytest.mark.parametrize("tc", [8, 16])
def test_host_converter_matches_oracle(tc):
    from graph_rws_amd.core import csr_to_bcsr_cpu
    g = synth.random_graph(333, 9.0, seed=5)
    win, cols, vals = csr_to_bcsr_cpu(g.num_nodes, g.row_ptr, g.col_idx, g.values, 16, tc)
    ow, oc, ov = oracle.csr_to_bcsr(g.num_nodes, g.row_ptr.numpy(), g.col_idx.numpy(),
                                    g.values.numpy(), 16, tc)
    np.testing.assert_array_equal(win.numpy(), ow)
    np.testing.assert_array_equal(cols.numpy(), oc)
    np.testing.assert_array_equal(vals.numpy(), ov.astype(np.float32))


def test_host_converter_rejects_bad_row_ptr():
    from graph_rws_amd.core import csr_to_bcsr_cpu
    rp = torch.tensor([0, 3, 2], dtype=torch.int64)
    with pytest.raises(RuntimeError, match="row_ptr decreases"):
        csr_to_bcsr_cpu(2, rp, torch.zeros(3, dtype=torch.int32), torch.ones(3), 16, 8)


def test_synthetic_config_shapes():
    g = synth.config_graph("c1")
    assert g.num_nodes == 2708 and g.nnz == 13264
    # symmetric with self loops, sym-normalised
    import scipy.sparse as sps
    A = sps.csr_matrix((g.values.numpy(), g.col_idx.numpy(), g.row_ptr.numpy()),
                       shape=(g.num_nodes, g.num_nodes))
    assert abs(A - A.T).max() < 1e-7
    assert np.all(A.diagonal() > 0)
    deg = np.diff(g.row_ptr.numpy())
    np.testing.assert_allclose(A.diagonal(), 1.0 / deg, rtol=1e-6)


def test_python_shim_keeps_reference_signatures():
    """The shim's ops take the reference's pybind11 argument names, in order,
    with the same defaults (core/wrapper/bind.cpp:99-159)."""
    import inspect
    import graph_rws_amd.core as core
    want = {
        "sample_all_layers": ["window_offset", "original_col_indices", "values_condensed",
                              "initial_seeds", "fanouts", "num_global_nodes", "static_scores",
                              "window_part_ids", "part_starts", "part_ends", "alpha", "beta",
                              "delta", "gamma_bonus", "score_scale", "use_hacs",
                              "locality_enabled", "tile_rows", "tile_cols", "warps_per_block"],
        "spmm_tc": ["window_offset", "original_col_indices", "values_condensed", "input_B",
                    "warps_per_block"],
        "spmm_transpose": ["window_offset", "original_col_indices", "values_condensed",
                           "grad_out", "num_cols"],
        "csr_to_bcsr_cpu": ["num_rows", "row_ptr", "col_idx", "values", "tile_rows", "tile_cols"],
        "reindex_bcsr": ["col_indices", "values_condensed", "active_windows", "tile_rows",
                         "tile_cols"],
    }
    defaults = {"sample_all_layers": dict(alpha=1.0, beta=10.0, delta=0.0, gamma_bonus=0.0,
                                          score_scale=100.0, use_hacs=0, locality_enabled=0,
                                          tile_rows=16, tile_cols=8, warps_per_block=8),
                "spmm_tc": dict(warps_per_block=8), "reindex_bcsr": dict(tile_rows=16, tile_cols=8)}
    for name, args in want.items():
        params = list(inspect.signature(getattr(core, name)).parameters.values())
        assert [p.name for p in params[:len(args)]] == args, name
        for k, v in defaults.get(name, {}).items():
            assert inspect.signature(getattr(core, name)).parameters[k].default == v, (name, k)
    t = core.SamplingTimingResult(1.0, 2.0, 3.0, 6.0)
    assert t.to_dict() == {"phase1_sampling_time": 1.0, "phase2_mapping_time": 2.0,
                           "phase3_recompression_time": 3.0, "total_time": 6.0}
    assert "SamplingTimingResult" in repr(t)


def test_window_sampler_host_checks_without_gpu():
    lib = L.load()
    assert lib.grws_window_sample_num(1) == 32 and lib.grws_window_sample_num(33) == 64
    assert lib.grws_window_sample_num(256) == 256
    n = ctypes.c_int64(-1)
    # empty inputs return before touching the device
    assert lib.grws_window_seeds(None, 0, 10, 16, 0, None, None, None, 0, ctypes.byref(n), None) == 0
    assert n.value == 0
    win = np.zeros(5, np.int64)  # never read: the fanout check comes first
    view = L.BcsrView(win.ctypes.data, None, None, 4, 0, 16, 8, 0, 0)
    T = ctypes.c_int64()
    off = np.zeros(1, np.int64)  # never written: the fanout check comes first
    st = lib.grws_window_topk(ctypes.byref(view), None, 0, 300, None, None, None,
                              off.ctypes.data, None, 0, ctypes.byref(T), None)
    assert st == -1 and b"fanout" in lib.grws_last_error()
    st = lib.grws_sample_hop(None, None, 10, 0, None, 5, 65, 42, None, None, None, 0, None, 0,
                             ctypes.byref(T), None)
    assert st == -1 and b"fanout" in lib.grws_last_error()
    st = lib.grws_sample_hop(None, None, 10, 0, None, 5, 8, 42, None, None, None, 39, None, 0,
                             ctypes.byref(T), None)
    assert st == -1 and b"edge_capacity" in lib.grws_last_error()


def test_aligned_rows_keeps_values_and_pads_pitch():
    from graph_rws_amd.data import aligned_rows
    x = torch.randn(7, 608).half()
    y = aligned_rows(x)
    assert y.stride() == (640, 1) and y.shape == x.shape and torch.equal(x, y)
    z = torch.randn(3, 256)  # 1024 B rows: already aligned, returned as is
    assert aligned_rows(z) is z


def test_packed_tiles_reject_bad_arguments_without_launching():
    """Packing needs 16x16 tiles of 16-bit values; grws_spmm_packed needs
    values of the x dtype and a sane value count.  All refused on the host."""
    lib = L.load()
    n = ctypes.c_int64()
    st = lib.grws_pack_tiles_count(None, None, 0, ctypes.byref(n), None)
    assert st == -1 and b"null graph" in lib.grws_last_error()
    view = L.BcsrView(None, None, None, 4, 10, 16, 8, L.GRWS_F16, 0)
    st = lib.grws_pack_tiles_count(ctypes.byref(view), None, 0, ctypes.byref(n), None)
    assert st == -1 and b"16x16" in lib.grws_last_error()
    view = L.BcsrView(None, None, None, 4, 10, 16, 16, L.GRWS_F32, 0)
    st = lib.grws_pack_tiles_count(ctypes.byref(view), None, 0, ctypes.byref(n), None)
    assert st == -2
    view = L.BcsrView(None, None, None, 4, 0, 16, 16, L.GRWS_F16, 0)  # no tiles: nothing to count
    assert lib.grws_pack_tiles_count(ctypes.byref(view), None, 0, ctypes.byref(n), None) == 0
    assert n.value == 0
    st = lib.grws_pack_tiles_fill(ctypes.byref(view), None, None, -1, None, 0, None)
    assert st == -1 and b"num_values" in lib.grws_last_error()
    assert lib.grws_pack_tiles_workspace_bytes(-1) == 0
    assert lib.grws_pack_tiles_workspace_bytes(1000) > 1000 * 12
    # grws_spmm_packed: f32 values with packed tiles, and a negative value count
    pk = L.PackedTilesView(None, None, 0)
    view = L.BcsrView(None, None, None, 4, 10, 16, 16, L.GRWS_F32, 0)
    st = lib.grws_spmm_packed(ctypes.byref(view), ctypes.byref(pk), None, None, L.GRWS_F16, 0, 8, 8, None,
                              L.GRWS_F16, 8, None, 0, None)
    assert st == -1 and b"packed tiles need" in lib.grws_last_error()
    pk = L.PackedTilesView(None, None, -5)
    view = L.BcsrView(None, None, None, 4, 10, 16, 16, L.GRWS_F16, 0)
    st = lib.grws_spmm_packed(ctypes.byref(view), ctypes.byref(pk), None, None, L.GRWS_F16, 0, 8, 8, None,
                              L.GRWS_F16, 8, None, 0, None)
    assert st == -1 and b"num_values" in lib.grws_last_error()


def test_spmm_residual_rejects_bad_arguments_without_launching():
    """grws_spmm_residual checks the residual's leading dimension and row
    count before anything touches the device."""
    lib = L.load()
    view = L.BcsrView(None, None, None, 1, 0, 16, 16, L.GRWS_F16, 0)
    r = ctypes.c_void_p(16)
    st = lib.grws_spmm_residual(ctypes.byref(view), None, None, None, L.GRWS_F16, 0, 8, 8, r, 4, 16, None,
                                L.GRWS_F16, 8, None, 0, None)
    assert st == L.GRWS_E_INVALID and b"ldr" in lib.grws_last_error()
    st = lib.grws_spmm_residual(ctypes.byref(view), None, None, None, L.GRWS_F16, 0, 8, 8, r, 8, -1, None,
                                L.GRWS_F16, 8, None, 0, None)
    assert st == L.GRWS_E_INVALID



def test_spmm_grouped_rejects_bad_arguments_without_launching():
    """grws_spmm_grouped validates the graph, the grouped tiles and X before
    anything touches the device: dtypes, group size, group count, X wider
    than the grouped columns, ldy, 16-byte rows, the value count."""
    lib = L.load()
    view = L.BcsrView(None, None, None, 8, 0, 16, 16, L.GRWS_F16, 0)  # 8 windows
    x = ctypes.c_void_p(256)  # never dereferenced: every case fails a check first

    def call(gt, x_dtype=L.GRWS_F16, x_rows=100, ldx=64, n=64, y_dtype=L.GRWS_F16, ldy=64, A=view):
        return lib.grws_spmm_grouped(ctypes.byref(A) if A is not None else None,
                                     ctypes.byref(gt) if gt is not None else None, x, x_dtype, x_rows, ldx, n,
                                     None, 0, 0, x, y_dtype, ldy, None)

    def gview(groups=2, slabs=0, values=0, mx=0, cols=100, G=4):
        # a group_offset address that no case reaches (every one fails a check first)
        return L.GroupedTilesView(ctypes.c_void_p(512), None, None, None, groups, slabs, values, mx, cols, G)

    assert call(None) == L.GRWS_E_INVALID and b"null" in lib.grws_last_error()
    assert call(gview(), x_dtype=L.GRWS_F32) == L.GRWS_E_DTYPE
    assert call(gview(), y_dtype=L.GRWS_BF16) == L.GRWS_E_DTYPE
    assert call(gview(G=3)) == L.GRWS_E_INVALID and b"group_size" in lib.grws_last_error()
    assert call(gview(groups=3)) == L.GRWS_E_INVALID and b"groups" in lib.grws_last_error()
    assert call(gview(cols=50)) == L.GRWS_E_INVALID and b"grouped for" in lib.grws_last_error()
    assert call(gview(values=1 << 31)) == L.GRWS_E_INVALID and b"too many values" in lib.grws_last_error()
    assert call(gview(), ldy=32) == L.GRWS_E_INVALID and b"ldy" in lib.grws_last_error()
    assert call(gview(), n=60, ldx=64, ldy=64) == L.GRWS_E_INVALID and b"16-byte rows" in lib.grws_last_error()


@pytest.mark.parametrize("name", [b"GRWS_GRP_K32", b"GRWS_GRP_DMA"])
def test_grouped_slab_pair_switches_round_trip(name):
    """GRWS_GRP_K32 (4-window groups on slab pairs, the default; 0 = single
    slabs) and GRWS_GRP_DMA (slab pairs staged by direct loads into LDS, the
    default; 0 = through registers) are tuning overrides like the others:
    unset reads -1, a set value reads back, -1 clears it, an unknown name is
    refused."""
    lib = L.load()
    assert lib.grws_spmm_get_tuning(name) == -1
    assert lib.grws_spmm_set_tuning(name, 0) == 0
    assert lib.grws_spmm_get_tuning(name) == 0
    assert lib.grws_spmm_set_tuning(name, -1) == 0
    assert lib.grws_spmm_get_tuning(name) == -1
    assert lib.grws_spmm_set_tuning(b"GRWS_NO_SUCH_SWITCH", 1) != 0
