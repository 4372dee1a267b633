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
