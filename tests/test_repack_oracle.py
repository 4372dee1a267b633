"""The repack restatement (oracle.repack_subgraph, sampler/sampler.py:420-690)
pinned by a hand-worked answer and by edge-set equality with the dense
matrix of the original graph."""
import numpy as np
import pytest

import oracle


def _bcsr_from_edges(n, edges, tile_cols, n_windows=None):
    rows = np.array([e[0] for e in edges], np.int64)
    cols = np.array([e[1] for e in edges], np.int64)
    vals = np.array([e[2] for e in edges], np.float32)
    order = np.lexsort((cols, rows))
    rows, cols, vals = rows[order], cols[order], vals[order]
    rp = np.zeros(n + 1, np.int64)
    np.add.at(rp, rows + 1, 1)
    rp = np.cumsum(rp)
    return oracle.csr_to_bcsr(n, rp, cols.astype(np.int32), vals, 16, tile_cols)


EDGES = [(0, 1, 1.0), (0, 20, 2.0), (0, 35, 3.0), (3, 25, 4.0), (33, 0, 5.0), (33, 20, 6.0),
         (33, 21, 7.0), (39, 39, 8.0), (17, 2, 9.0)]


def _dense_of(win, cols, vals, tc, n_rows_pad, n_cols):
    return oracle.bcsr_to_dense(win, cols, vals, 16, tc, n_cols)[:n_rows_pad]


@pytest.mark.parametrize("tc", [8, 16])
def test_known_answer_all_kept(tc):
    win, cols, vals = _bcsr_from_edges(40, EDGES, tc)
    r = oracle.repack_subgraph(win, cols, vals, 40, tc, [2, 5, 0, -1], ratio=5.0)
    assert r["window_ids"].tolist() == [0, 2]
    internal = list(range(16)) + list(range(32, 40))
    assert r["num_internal"] == 24
    assert r["input_nodes"].tolist() == internal + [20, 21, 25]
    D = _dense_of(r["window_offset"], r["halo_cols"], r["halo_values"], tc, 32, 27)
    want = np.zeros((32, 27))
    want[0, 1], want[0, 24], want[0, 19], want[3, 26] = 1, 2, 3, 4       # rows 0 and 3
    want[17, 0], want[17, 24], want[17, 25], want[23, 23] = 5, 6, 7, 8  # global 33 and 39
    np.testing.assert_array_equal(D, want)
    Di = _dense_of(r["window_offset"], r["inner_cols"], r["inner_values"], tc, 32, 24)
    np.testing.assert_array_equal(Di, want[:, :24])
    assert r["halo_nnz"] == 8 and r["inner_nnz"] == 4


def test_known_answer_over_budget():
    win, cols, vals = _bcsr_from_edges(40, EDGES, 8)
    # budget int(24 * 0.1) = 2 of the 3 candidates [20, 21, 25]; the draw keeps positions 2 and 0
    r = oracle.repack_subgraph(win, cols, vals, 40, 8, [0, 2], ratio=0.1, perm=[2, 0, 1])
    assert r["num_external"] == 3
    assert r["input_nodes"].tolist()[24:] == [20, 25]
    D = _dense_of(r["window_offset"], r["halo_cols"], r["halo_values"], 8, 32, 26)
    assert D[17, 25] == 0 and D[0, 24] == 2 and D[3, 25] == 4  # the edge to 21 is gone
    with pytest.raises(ValueError):
        oracle.repack_subgraph(win, cols, vals, 40, 8, [0, 2], ratio=0.1)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_edge_sets_match_dense_original(seed):
    rng = np.random.default_rng(seed)
    n = 300
    edges = {}
    for _ in range(3000):
        edges[(int(rng.integers(0, n)), int(rng.integers(0, n)))] = float(rng.integers(1, 9))
    win, cols, vals = _bcsr_from_edges(n, [(a, b, v) for (a, b), v in edges.items()], 16)
    A = oracle.bcsr_to_dense(win, cols, vals, 16, 16, n)
    wids = rng.choice(len(win) - 1, 6, replace=False)
    n_ext = oracle.repack_subgraph(win, cols, vals, n, 16, wids, 1e9)["num_external"]
    for ratio in (100.0, 0.5):
        nc = oracle.repack_subgraph(win, cols, vals, n, 16, wids, ratio, perm=rng.permutation(n_ext))
        inp = nc["input_nodes"]
        rows = (np.repeat(nc["window_ids"], 16) * 16 + np.tile(np.arange(16), len(wids)))
        D = _dense_of(nc["window_offset"], nc["halo_cols"], nc["halo_values"], 16, 16 * len(wids), inp.size)
        ok_rows = rows < n
        # every kept (row, column) pair carries the original value, every other is 0
        np.testing.assert_array_equal(D[ok_rows], A[rows[ok_rows]][:, inp])
        assert inp[: nc["num_internal"]].tolist() == rows[ok_rows].tolist()
        ext = inp[nc["num_internal"]:]
        assert np.all(np.diff(ext) > 0)
        Di = _dense_of(nc["window_offset"], nc["inner_cols"], nc["inner_values"], 16, 16 * len(wids),
                       nc["num_internal"])
        np.testing.assert_array_equal(Di[ok_rows], A[rows[ok_rows]][:, inp[: nc["num_internal"]]])
