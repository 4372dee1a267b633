"""The full-size checker (tests/_fullsize.py) can see a missing term.

On a c3-shaped graph (SBM, 483 non-zeros per row) at 2% of c3's size, an
output that is the exact product rounded once to f16 passes both tiers,
and one computed with a single non-zero of every window dropped (or one
added twice) fails the tight tier in every such row, although the 1e-2
contract bound alone lets most of those elements through.  The reference's
forward adds every stored tile (/root/reference/core/include/spmm_tc.cuh:
113-154): a kernel that skips a slab in some windows must not pass.  CPU
only (the oracle and numpy stand in for the device).
"""
import numpy as np
import pytest
import torch

import oracle
from _fullsize import DT, all_row_nnz, check_forward, flagged, tight_bound, window_row_nnz
from graph_rws_amd import synth


class _Host:
    def __init__(self, win, cols, vals, tc, n):
        self.win, self.cols, self.vals, self.vdt, self.tc = win, cols, vals, "f16", tc
        self.W = len(win) - 1
        self.num_cols = n


@pytest.fixture(scope="module")
def c3_small():
    g = synth.config_graph("c3", scale=0.02)
    n = g.num_nodes
    rp, ci = g.row_ptr.numpy(), g.col_idx.numpy()
    va = g.values.numpy().astype(np.float16).astype(np.float32)
    win, cols, vals = oracle.csr_to_bcsr(n, rp, ci, va, 16, 16)
    hg = _Host(win, cols, vals.astype(np.float16), 16, n)
    X = synth.features(n, 64, seed=3).half()
    return hg, X


def _product(hg, X, vals):
    Y, _ = oracle.bcsr_spmm(hg.win, hg.cols, vals.astype(np.float64), 16, hg.tc, X.double().numpy())
    return torch.from_numpy(Y).half()


def _drop_one_per_window(hg, seed, factor):
    """A copy of the values with one non-zero of every non-empty window
    scaled by `factor` (0: dropped, 2: added twice); returns (vals, rows)."""
    rng = np.random.default_rng(seed)
    v = hg.vals.astype(np.float32).copy()
    rows = []
    for w in range(hg.W):
        a, b = int(hg.win[w]), int(hg.win[w + 1])
        nz = np.flatnonzero(v[a * 256:b * 256])
        if nz.size == 0:
            continue
        j = a * 256 + int(rng.choice(nz))
        v[j] *= factor
        rows.append(16 * w + (j % 256) // 16)
    return v, np.asarray(rows)


def test_exact_product_passes_both_tiers(c3_small):
    hg, X = c3_small
    Y = _product(hg, X, hg.vals)
    st = check_forward(hg, X, Y, 1e-2, seed=1)
    assert st["worst_of_tight"] <= 1.0 and st["worst_of_contract"] < 0.1


@pytest.mark.parametrize("factor", [0.0, 2.0])
def test_one_term_per_window_is_flagged(c3_small, factor):
    hg, X = c3_small
    v, rows = _drop_one_per_window(hg, seed=5, factor=factor)
    Yb = _product(hg, X, v)
    # every window against the true product, both tiers
    sel = np.arange(hg.W)
    Yr, Ya = oracle.bcsr_spmm_windows(hg.win, hg.cols, hg.vals, "f16", hg.tc, X.numpy(), "f16", sel)
    err = np.abs(Yb.double().numpy() - Yr)
    k = window_row_nnz(hg, sel)[:, None]
    tight = flagged(err, tight_bound(Yr, Ya, k, "f16", "f16", "f16"))
    contract = flagged(err, 1e-2 * Ya)
    # every changed row is flagged in (nearly) every one of its 64 columns
    per_row = (err > tight_bound(Yr, Ya, k, "f16", "f16", "f16"))[rows].sum(axis=1)
    assert per_row.min() >= 48, per_row.min()
    assert tight >= 0.9 * 64 * rows.size
    assert contract < 0.1 * tight, (contract, tight)
    # and check_forward itself fails, on its own window sample and projection
    with pytest.raises(AssertionError, match="tight tier"):
        check_forward(hg, X, Yb, 1e-2, seed=1)


def test_row_counts_match_the_csr(c3_small):
    hg, _ = c3_small
    k = all_row_nnz(hg)
    n = hg.num_cols
    dense_nnz = np.zeros(16 * hg.W, np.int64)
    for w in range(hg.W):
        a, b = int(hg.win[w]), int(hg.win[w + 1])
        t = hg.vals[a * 256:b * 256].reshape(-1, 16, 16)
        dense_nnz[16 * w:16 * w + 16] = (t != 0).sum(axis=(0, 2))
    np.testing.assert_array_equal(k, dense_nnz)
    assert k[:n].sum() == np.count_nonzero(hg.vals)
    assert DT[torch.float16] == hg.vdt
