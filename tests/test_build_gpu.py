"""Device BCSR build (COO/CSR -> BCSR, transpose, COO -> CSR) and reindex on
the GPU.  Integer and index results must be bit-exact against the oracle /
host converter; float32 values are moved, never computed, so they are
bit-exact too; float16/bfloat16 values equal torch's round-to-nearest-even
cast of the float32 values."""
import numpy as np
import pytest
import scipy.sparse as sps
import torch

import oracle
from graph_rws_amd import builder, core, synth
from graph_rws_amd.core._lib import GrwsError

pytestmark = pytest.mark.gpu


def _host(g, tc):
    return core.csr_to_bcsr_cpu(g.num_nodes, g.row_ptr, g.col_idx, g.values, 16, tc)


def _eq(a, b):
    assert torch.equal(a.cpu(), b.cpu())


def _oracle_bcsr(g, tc):
    """The oracle's restatement of convert_wrapper.cpp:27-180 (itself pinned
    to the reference's compiled converter in tests/test_oracle.py)."""
    ow, oc, ov = oracle.csr_to_bcsr(g.num_nodes, g.row_ptr.numpy(), g.col_idx.numpy(), g.values.numpy(), 16, tc)
    return torch.from_numpy(ow), torch.from_numpy(oc), torch.from_numpy(ov.astype(np.float32))


GRAPHS = {
    "random": lambda: synth.random_graph(777, 11.0, seed=3),
    "powerlaw": lambda: synth.chung_lu(5000, 80000, 2.1, seed=4),
    "tiny": lambda: synth.random_graph(5, 2.0, seed=1),
}


@pytest.mark.parametrize("name", list(GRAPHS))
@pytest.mark.parametrize("tc", [8, 16])
@pytest.mark.parametrize("vdt", [torch.float32, torch.float16, torch.bfloat16])
def test_csr_build_matches_oracle(cuda_device, name, tc, vdt):
    """The device build equals the oracle's converter and the host one."""
    print(f"case build {name} tc={tc} {vdt}", flush=True)
    g = GRAPHS[name]()
    ow, oc, ov = _oracle_bcsr(g, tc)
    hw, hc, hv = _host(g, tc)
    dw, dc, dv = builder.csr_to_bcsr_device(g.num_nodes, g.num_nodes, g.row_ptr.to(cuda_device),
                                            g.col_idx.to(cuda_device), g.values.to(cuda_device),
                                            tile_cols=tc, values_dtype=vdt)
    torch.cuda.synchronize()
    _eq(dw, ow)
    _eq(dc, oc)
    assert dv.dtype == vdt
    _eq(dv, ov.to(vdt))
    _eq(hw, ow)
    _eq(hc, oc)
    _eq(hv, ov)


def test_coo_build_duplicates_last_wins(cuda_device):
    """Duplicate (row, col) edges: the last in input order wins
    (convert_wrapper.cpp:174), as in the oracle's restatement."""
    print("case duplicates", flush=True)
    rng = np.random.default_rng(11)
    n = 300
    rows = rng.integers(0, n, 6000).astype(np.int32)
    cols = rng.integers(0, n, 6000).astype(np.int32)
    vals = rng.standard_normal(6000).astype(np.float32)
    # CSR in input order within each row (stable by row) = the oracle's CSR order
    order = np.argsort(rows, kind="stable")
    rp = np.zeros(n + 1, np.int64)
    np.add.at(rp, rows + 1, 1)
    rp = np.cumsum(rp)
    ow, oc, ov = oracle.csr_to_bcsr(n, rp, cols[order], vals[order], 16, 16)
    dw, dc, dv = builder.coo_to_bcsr_device(n, n, torch.from_numpy(rows).to(cuda_device),
                                            torch.from_numpy(cols).to(cuda_device),
                                            torch.from_numpy(vals).to(cuda_device), tile_cols=16)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dw.cpu().numpy(), ow)
    np.testing.assert_array_equal(dc.cpu().numpy(), oc)
    np.testing.assert_array_equal(dv.cpu().numpy(), ov.astype(np.float32))


def _window_case_csr(hub: bool, seed: int):
    """A 75-row CSR (five 16-row windows, the last ragged) over 2^20 + 5
    columns: window 0 holds 8,000 edges over 3,000 columns (many duplicate
    (row, column) edges), window 1 holds 11,200 edges over all the columns
    (span above 2^18), window 2 one column only, window 3 none, window 4 a
    few short rows; rows are unsorted.  hub adds 20,000 edges to row 40 and
    3,000 over 100 columns to row 41 (a window above 16,384 edges, with
    duplicates)."""
    rng = np.random.default_rng(seed)
    n_r, n_c = 75, (1 << 20) + 5
    per_row = []
    for r in range(n_r):
        if r < 16:
            c = rng.integers(0, 3000, 500)
        elif r < 32:
            c = rng.integers(0, n_c, 700)
        elif r < 48:
            c = np.full(10, 7)
        elif r < 64:
            c = np.zeros(0, np.int64)
        else:
            c = rng.integers(0, n_c, int(rng.integers(0, 40)))
        if hub and r == 40:
            c = rng.integers(0, n_c, 20000)
        if hub and r == 41:  # many duplicate (row, column) edges in the same large window
            c = rng.integers(0, 100, 3000)
        per_row.append(c.astype(np.int32))
    rp = np.zeros(n_r + 1, np.int64)
    rp[1:] = np.cumsum([len(c) for c in per_row])
    cols = np.concatenate(per_row)
    vals = rng.standard_normal(cols.size).astype(np.float32)
    return n_r, n_c, rp, cols, vals


@pytest.mark.parametrize("hub", [False, True])
@pytest.mark.parametrize("tc", [8, 16])
@pytest.mark.parametrize("vdt", [torch.float32, torch.float16, torch.bfloat16])
def test_csr_build_window_paths(cuda_device, hub, tc, vdt):
    """CSR input through each case of the window-by-window build (hub: a
    window above 16,384 edges, sorted in global scratch by one work-group):
    equal to the oracle's converter, duplicates last-wins, values bit-exact
    (f32) or its round-to-nearest-even cast (f16, bf16)."""
    print(f"case window paths hub={hub} tc={tc} {vdt}", flush=True)
    n_r, n_c, rp, cols, vals = _window_case_csr(hub, seed=21 + tc)
    ow, oc, ov = oracle.csr_to_bcsr(n_r, rp, cols, vals, 16, tc)
    dw, dc, dv = builder.csr_to_bcsr_device(n_r, n_c, torch.from_numpy(rp).to(cuda_device),
                                            torch.from_numpy(cols).to(cuda_device),
                                            torch.from_numpy(vals).to(cuda_device), tile_cols=tc,
                                            values_dtype=vdt)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dw.cpu().numpy(), ow)
    np.testing.assert_array_equal(dc.cpu().numpy(), oc)
    _eq(dv, torch.from_numpy(ov.astype(np.float32)).to(vdt))


def test_build_under_capture_is_refused_cleanly(cuda_device):
    """The build waits for its data-dependent sizes, which a stream under
    capture does not allow.  Inside a capture it returns a clean error
    before it touches the stream, so the capture stays valid (it ends, and
    its replays run the work captured around the call), and the same build
    then runs eagerly and equals the oracle's converter."""
    print("case build under capture", flush=True)
    g = GRAPHS["random"]()
    args = [t.to(cuda_device) for t in (g.row_ptr, g.col_idx, g.values)]
    x = torch.zeros(64, device=cuda_device)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, capture_error_mode="thread_local"):
        x.add_(1.0)
        with pytest.raises(GrwsError, match="being captured"):
            builder.csr_to_bcsr_device(g.num_nodes, g.num_nodes, *args, tile_cols=16)
        x.mul_(3.0)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
    assert float(x[0]) == 39.0 and bool((x == x[0]).all())  # ((0 + 1) 3 + 1) 3 + 1) 3
    dw, dc, dv = builder.csr_to_bcsr_device(g.num_nodes, g.num_nodes, *args, tile_cols=16)
    ow, oc, ov = _oracle_bcsr(g, 16)
    _eq(dw, ow)
    _eq(dc, oc)
    _eq(dv, ov)


def test_big_window_builds_on_concurrent_streams(cuda_device):
    """Windows above 16,384 edges run on one extra stream per device, forked
    from and joined back into the caller's stream.  Two threads, each on a
    stream of its own, build graphs with such windows at the same time (a
    CSR build and a transposed one, three times each): every result equals
    the oracle's converter."""
    import threading
    print("case big windows on concurrent streams", flush=True)
    n_r, n_c, rp, cols, vals = _window_case_csr(True, seed=51)
    want_csr = oracle.csr_to_bcsr(n_r, rp, cols, vals, 16, 16)
    # transposed: 17,000 rows, each with an edge to column 3 (a window of A^T above 16,384 edges) and a random one
    rng = np.random.default_rng(5)
    t_rows = 17000
    t_cols = np.stack([np.full(t_rows, 3), rng.integers(0, n_c, t_rows)], 1).reshape(-1).astype(np.int32)
    t_vals = rng.standard_normal(t_cols.size).astype(np.float32)
    t_rp = 2 * np.arange(t_rows + 1, dtype=np.int64)
    want_t = _oracle_transposed(t_rows, n_c, t_rp, t_cols, t_vals, 16)
    got, failures = {}, []

    def run(name, nr, rp_, cols_, vals_, transpose):
        try:
            s = torch.cuda.Stream(device=cuda_device)
            with torch.cuda.stream(s):
                args = [torch.from_numpy(a).to(cuda_device, non_blocking=False) for a in (rp_, cols_, vals_)]
                out = []
                for _ in range(3):
                    w, c, v = builder.csr_to_bcsr_device(nr, n_c, *args, tile_cols=16,
                                                         values_dtype=torch.float32, transpose=transpose)
                    out.append((w, c, v))
                s.synchronize()
                got[name] = [(w.cpu().numpy(), c.cpu().numpy(), v.cpu().numpy()) for w, c, v in out]
        except BaseException as e:  # reported by the main thread
            failures.append(e)

    threads = [threading.Thread(target=run, args=("csr", n_r, rp, cols, vals, False)),
               threading.Thread(target=run, args=("t", t_rows, t_rp, t_cols, t_vals, True))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=90)
        assert not t.is_alive(), "a build thread did not finish"
    assert not failures, failures
    for name, want in (("csr", want_csr), ("t", want_t)):
        for w, c, v in got[name]:
            np.testing.assert_array_equal(w, want[0])
            np.testing.assert_array_equal(c, want[1])
            np.testing.assert_array_equal(v, want[2].astype(np.float32))


def _boundary_csr(seed: int):
    """One 16-row window per size class edge -- 2,048 / 2,049, 8,192 / 8,193,
    16,384 / 16,385 edges -- each with a column span exactly filling or just
    past its class's bitmap (2^16, 2^18, 2^19 columns), duplicates included."""
    rng = np.random.default_rng(seed)
    # (edges, columns spanned): a span of 2^k columns fills a 2^k-bit bitmap
    # exactly, 2^k + 1 takes the class's radix sort instead
    sizes = [(2048, 1 << 16), (2048, (1 << 16) + 1), (2049, 1 << 18), (8192, (1 << 18) + 1),
             (8193, 1 << 19), (16384, (1 << 19) + 1), (16385, 1 << 19), (8192, 1 << 18)]
    n_c = (1 << 19) + 8
    per_row = []
    for m, span in sizes:
        base = int(rng.integers(0, n_c - span))
        c = base + rng.integers(0, span, m)
        c[0], c[1] = base, base + span - 1  # the span's two ends
        c[2:40] = c[40:78]  # duplicates
        split = np.sort(rng.integers(0, m, 15))
        per_row += [p.astype(np.int32) for p in np.split(c, split)]
    rp = np.zeros(len(per_row) + 1, np.int64)
    rp[1:] = np.cumsum([len(c) for c in per_row])
    cols = np.concatenate(per_row)
    vals = rng.standard_normal(cols.size).astype(np.float32)
    return len(per_row), n_c, rp, cols, vals


@pytest.mark.parametrize("transpose", [False, True])
def test_build_size_and_span_boundaries(cuda_device, transpose):
    """Windows at every size-class edge of the window-by-window build, with
    column spans at the edges of each class's bitmap: equal to the oracle's
    converter (transposed: over A^T)."""
    print(f"case size/span boundaries transpose={transpose}", flush=True)
    n_r, n_c, rp, cols, vals = _boundary_csr(seed=77)
    if transpose:
        ow, oc, ov = _oracle_transposed(n_r, n_c, rp, cols, vals, 16)
    else:
        ow, oc, ov = oracle.csr_to_bcsr(n_r, rp, cols, vals, 16, 16)
    dw, dc, dv = builder.csr_to_bcsr_device(n_r, n_c, torch.from_numpy(rp).to(cuda_device),
                                            torch.from_numpy(cols).to(cuda_device),
                                            torch.from_numpy(vals).to(cuda_device), tile_cols=16,
                                            transpose=transpose)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dw.cpu().numpy(), ow)
    np.testing.assert_array_equal(dc.cpu().numpy(), oc)
    np.testing.assert_array_equal(dv.cpu().numpy(), ov.astype(np.float32))


def _oracle_transposed(n_r, n_c, rp, cols, vals, tc):
    """BCSR of A^T by the oracle's converter over A^T's CSR, whose rows list
    their edges in input order (a stable sort by column), so duplicate
    edges keep their input order."""
    rows = np.repeat(np.arange(n_r, dtype=np.int32), np.diff(rp))
    order = np.argsort(cols, kind="stable")
    trp = np.zeros(n_c + 1, np.int64)
    np.add.at(trp, cols.astype(np.int64) + 1, 1)
    return oracle.csr_to_bcsr(n_c, np.cumsum(trp), rows[order], vals[order], 16, tc)


@pytest.mark.parametrize("hub", [False, True])
@pytest.mark.parametrize("tc", [8, 16])
@pytest.mark.parametrize("vdt", [torch.float32, torch.bfloat16])
def test_transposed_csr_build_window_paths(cuda_device, hub, tc, vdt):
    """Transposed builds from a CSR: windows of A^T grouped by a sort over
    the window bits, then built window by window; hub: a column of 17,000
    in-edges (a window above 16,384 edges), a tenth of them duplicated.
    Equal to the oracle's converter over A^T, duplicates in input order."""
    print(f"case transposed window paths hub={hub} tc={tc} {vdt}", flush=True)
    n_r, n_c, rp, cols, vals = _window_case_csr(False, seed=40 + tc)
    if hub:  # 17,000 more rows, each with an edge to column 3 and one random edge (a tenth: column 3 again)
        rng = np.random.default_rng(3)
        other = np.where(rng.random(17000) < 0.1, 3, rng.integers(0, n_c, 17000))
        extra = np.stack([np.full(17000, 3), other], 1).reshape(-1).astype(np.int32)
        cols = np.concatenate([cols, extra])
        vals = np.concatenate([vals, rng.standard_normal(extra.size).astype(np.float32)])
        rp = np.concatenate([rp, rp[-1] + 2 * np.arange(1, 17001, dtype=np.int64)])
        n_r += 17000
    ow, oc, ov = _oracle_transposed(n_r, n_c, rp, cols, vals, tc)
    dw, dc, dv = builder.csr_to_bcsr_device(n_r, n_c, torch.from_numpy(rp).to(cuda_device),
                                            torch.from_numpy(cols).to(cuda_device),
                                            torch.from_numpy(vals).to(cuda_device), tile_cols=tc, transpose=True,
                                            values_dtype=vdt)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dw.cpu().numpy(), ow)
    np.testing.assert_array_equal(dc.cpu().numpy(), oc)
    _eq(dv, torch.from_numpy(ov.astype(np.float32)).to(vdt))


def test_coo_build_wide_columns_global_sort(cuda_device):
    """COO input over more than 2^27 columns (beyond the window-by-window
    path's column span): the global sort, equal to the oracle."""
    print("case coo wide columns", flush=True)
    rng = np.random.default_rng(17)
    n, n_c, m = 300, (1 << 27) + 100, 6000
    rows = rng.integers(0, n, m).astype(np.int32)
    cols = rng.integers(0, n_c, m).astype(np.int32)
    cols[:50] = n_c - 1
    vals = rng.standard_normal(m).astype(np.float32)
    order = np.argsort(rows, kind="stable")
    rp = np.zeros(n + 1, np.int64)
    np.add.at(rp, rows + 1, 1)
    ow, oc, ov = oracle.csr_to_bcsr(n, np.cumsum(rp), cols[order], vals[order], 16, 16)
    dw, dc, dv = builder.coo_to_bcsr_device(n, n_c, torch.from_numpy(rows).to(cuda_device),
                                            torch.from_numpy(cols).to(cuda_device),
                                            torch.from_numpy(vals).to(cuda_device), tile_cols=16)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dw.cpu().numpy(), ow)
    np.testing.assert_array_equal(dc.cpu().numpy(), oc)
    np.testing.assert_array_equal(dv.cpu().numpy(), ov.astype(np.float32))


@pytest.mark.parametrize("vdt", [torch.float32, torch.float16])
def test_csr_build_unaligned_outputs(cuda_device, vdt):
    """Outputs that start one element past a 16-byte boundary (a C-ABI
    caller's buffers): the window-by-window fill stores element by element
    and gives the same BCSR."""
    import ctypes
    from graph_rws_amd.core import _lib as L
    print(f"case unaligned outputs {vdt}", flush=True)
    n_r, n_c, rp, cols, vals = _window_case_csr(False, seed=5)
    ow, oc, ov = oracle.csr_to_bcsr(n_r, rp, cols, vals, 16, 16)
    d_rp, d_c, d_v = (torch.from_numpy(a).to(cuda_device) for a in (rp, cols, vals))
    W = (n_r + 15) // 16
    win = torch.empty(W + 1, dtype=torch.int64, device=cuda_device)
    wsb = int(L.load().grws_bcsr_build_workspace_bytes(cols.size, n_r, n_c, 0))
    ws = torch.empty(wsb, dtype=torch.uint8, device=cuda_device)
    T = ctypes.c_int64()
    stream = L.stream_of(cuda_device)
    L.call("grws_bcsr_build_count", L.ptr(d_rp), None, L.ptr(d_c), L.ptr(d_v), cols.size, n_r, n_c, 16, 0,
           L.ptr(win), L.ptr(ws), wsb, ctypes.byref(T), stream)
    T = T.value
    cbuf = torch.empty(T * 16 + 1, dtype=torch.int32, device=cuda_device)
    vbuf = torch.empty(T * 256 + 1, dtype=vdt, device=cuda_device)
    L.call("grws_bcsr_build_fill", cols.size, n_r, n_c, 16, 0, L.ptr(win), T, L.ptr(cbuf[1:]), L.ptr(vbuf[1:]),
           L.dtype_code(vdt), L.ptr(ws), wsb, stream)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(win.cpu().numpy(), ow)
    np.testing.assert_array_equal(cbuf[1:].cpu().numpy(), oc)
    _eq(vbuf[1:], torch.from_numpy(ov.astype(np.float32)).to(vdt))


def test_rectangular_and_empty(cuda_device):
    print("case rectangular", flush=True)
    # 37 rows x 1000 cols, rows 0..15 empty
    rng = np.random.default_rng(2)
    rows = rng.integers(16, 37, 400).astype(np.int32)
    cols = rng.integers(0, 1000, 400).astype(np.int32)
    vals = np.ones(400, np.float32)
    order = np.argsort(rows, kind="stable")
    rp = np.zeros(38, np.int64)
    np.add.at(rp, rows + 1, 1)
    rp = np.cumsum(rp)
    ow, oc, ov = oracle.csr_to_bcsr(37, rp, cols[order], vals[order], 16, 8)
    dw, dc, dv = builder.csr_to_bcsr_device(37, 1000, torch.from_numpy(rp).to(cuda_device),
                                            torch.from_numpy(cols[order]).to(cuda_device),
                                            torch.from_numpy(vals[order]).to(cuda_device), tile_cols=8)
    np.testing.assert_array_equal(dw.cpu().numpy(), ow)
    np.testing.assert_array_equal(dc.cpu().numpy(), oc)
    assert ow[1] == 0  # first window empty
    # no edges at all
    rp0 = torch.zeros(21, dtype=torch.int64, device=cuda_device)
    ew, ec, ev = builder.csr_to_bcsr_device(20, 20, rp0, torch.empty(0, dtype=torch.int32, device=cuda_device),
                                            None, tile_cols=16)
    assert ew.cpu().tolist() == [0, 0, 0] and ec.numel() == 0 and ev.numel() == 0


def test_build_rejects_out_of_range(cuda_device):
    print("case build errors", flush=True)
    rp = torch.tensor([0, 2, 3], dtype=torch.int64, device=cuda_device)
    ci = torch.tensor([0, 5, 1], dtype=torch.int32, device=cuda_device)
    with pytest.raises(GrwsError, match="column index is out of range"):
        builder.csr_to_bcsr_device(2, 4, rp, ci, None, tile_cols=8)
    bad = torch.tensor([0, 3, 2], dtype=torch.int64, device=cuda_device)
    with pytest.raises(GrwsError, match="row_ptr"):
        builder.csr_to_bcsr_device(2, 4, bad, ci.clamp(max=3), None, tile_cols=8)


@pytest.mark.parametrize("n_r,n_c,m", [(500, 900, 20000), (1, 7, 3), (16384, 50, 40000),
                                       (16385, 50, 40000), (4096 * 1024, 30, 300000),
                                       (4096 * 1024 + 1, 30, 300000), (5000000, 1000, 6000000)])
def test_coo_to_csr_matches_stable_sort(cuda_device, n_r, n_c, m):
    """Row pointers are an exclusive scan over n_r counts: the sizes cover a
    one-launch scan (up to 16,384), the two-launch scan (up to 1,024 tiles of
    4,096) and the three-launch scan beyond, at their boundaries."""
    print(f"case coo_to_csr {n_r}x{n_c} m={m}", flush=True)
    rng = np.random.default_rng(5)
    src = rng.integers(0, n_r, m).astype(np.int32)
    dst = rng.integers(0, n_c, m).astype(np.int32)
    w = rng.standard_normal(m).astype(np.float32)
    E, rp, ci, va = builder.coo_to_csr_device(n_r, n_c, torch.from_numpy(src).to(cuda_device),
                                              torch.from_numpy(dst).to(cuda_device),
                                              torch.from_numpy(w).to(cuda_device))
    order = np.lexsort((dst, src))  # stable: by src, then dst, ties in input order
    exp_rp = np.concatenate([[0], np.cumsum(np.bincount(src, minlength=n_r))])
    assert E == m
    np.testing.assert_array_equal(rp.cpu().numpy(), exp_rp)
    np.testing.assert_array_equal(ci.cpu().numpy(), dst[order])
    np.testing.assert_array_equal(va.cpu().numpy(), w[order])


def _coo_of_bcsr(win, cols, vals, tc, num_cols):
    """COO of BCSR arrays in the order grws_bcsr_to_coo emits: tile by tile,
    each tile's slots in (row, column) order, keeping slots whose column is
    in [0, num_cols) and whose value is nonzero."""
    T = cols.size // tc
    tile_win = np.repeat(np.arange(win.size - 1), np.diff(win))
    s = np.arange(16 * tc)
    row = (16 * tile_win[:, None] + s[None, :] // tc).reshape(-1)
    col = cols.reshape(T, tc)[:, s % tc].reshape(-1)
    val = vals.reshape(-1).astype(np.float32)
    keep = (col >= 0) & (col < num_cols) & (val != 0)
    return row[keep], col[keep], val[keep]


@pytest.mark.parametrize("tc", [8, 16])
@pytest.mark.parametrize("vdt", [torch.float32, torch.float16])
@pytest.mark.parametrize("offset", [0, 1])
def test_bcsr_to_coo_matches_slot_order(cuda_device, tc, vdt, offset):
    """BCSR -> COO on the device: every valid nonzero slot, in tile and slot
    order; values one element past a 16-byte boundary (offset 1) take the
    value-by-value loads."""
    print(f"case bcsr_to_coo tc={tc} {vdt} offset={offset}", flush=True)
    g = synth.chung_lu(3000, 50000, 2.1, seed=12)
    hw, hc, hv = _host(g, tc)
    hv = hv.to(vdt)
    hv.view(-1)[::7] = 0  # explicit zeros are dropped
    buf = torch.empty(hv.numel() + offset, dtype=vdt, device=cuda_device)
    dv = buf[offset:]
    dv.copy_(hv.view(-1).to(cuda_device))
    r, c, v = builder.bcsr_to_coo(hw.to(cuda_device), hc.to(cuda_device), dv, tc, g.num_nodes - 5)
    torch.cuda.synchronize()
    er, ec, ev = _coo_of_bcsr(hw.numpy(), hc.numpy(), hv.float().numpy(), tc, g.num_nodes - 5)
    np.testing.assert_array_equal(r.cpu().numpy(), er)
    np.testing.assert_array_equal(c.cpu().numpy(), ec)
    np.testing.assert_array_equal(v.cpu().numpy(), ev)


@pytest.mark.parametrize("tc", [8, 16])
def test_transpose_matches_host_build_of_transpose(cuda_device, tc):
    """BCSR(A^T) built from BCSR(A) on the device equals the host converter
    run on scipy's CSR transpose."""
    print(f"case transpose tc={tc}", flush=True)
    g = synth.chung_lu(3000, 50000, 2.1, seed=8)
    n = g.num_nodes
    hw, hc, hv = _host(g, tc)
    tw, tcol, tv = builder.transpose_arrays(hw.to(cuda_device), hc.to(cuda_device),
                                            hv.to(cuda_device), tc, n)
    W = hw.numel() - 1
    A = sps.csr_matrix((g.values.numpy(), g.col_idx.numpy(), g.row_ptr.numpy()), shape=(n, n))
    AT = A.T.tocsr()
    AT.sort_indices()
    ew, ec, ev = core.csr_to_bcsr_cpu(n, torch.from_numpy(AT.indptr.astype(np.int64)),
                                      torch.from_numpy(AT.indices.astype(np.int32)),
                                      torch.from_numpy(AT.data.astype(np.float32)), 16, tc)
    _eq(tw, ew)
    _eq(tcol, ec)
    _eq(tv, ev)
    assert W * 16 >= n


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16])
def test_spmm_transpose_parity(cuda_device, xdt):
    """A^T G through the cached transpose against the float64 oracle
    (spmm_tc.cuh:238-269 semantics), rtol 1e-5 (f32) / 1e-2 (f16, bf16)."""
    print(f"case spmm_transpose {xdt}", flush=True)
    rtol = 1e-5 if xdt == torch.float32 else 1e-2
    g = synth.chung_lu(2000, 30000, 2.1, seed=9)
    for tc in (8, 16):
        w, c, v = _host(g, tc)
        w, c = w.to(cuda_device), c.to(cuda_device)
        v = v.to(cuda_device).to(xdt)
        W = w.numel() - 1
        G = synth.features(16 * W, 72, seed=3, device=cuda_device).to(xdt)
        out = core.spmm_transpose(w, c, v, G, g.num_nodes, tile_cols=tc)
        out2 = core.spmm_transpose(w, c, v, G, g.num_nodes, tile_cols=tc)
        torch.cuda.synchronize()
        assert out.shape == (g.num_nodes, 72)
        assert torch.equal(out.view(-1).view(torch.int16 if xdt != torch.float32 else torch.int32),
                           out2.view(-1).view(torch.int16 if xdt != torch.float32 else torch.int32))
        ref, refa = oracle.bcsr_spmm_t(w.cpu().numpy(), c.cpu().numpy(), v.double().cpu().numpy(),
                                       16, tc, G.double().cpu().numpy(), g.num_nodes)
        err = np.abs(out.double().cpu().numpy() - ref)
        assert np.all(err <= rtol * refa), f"max excess {(err - rtol * refa).max():.3e}"


@pytest.mark.parametrize("vdt", [torch.float32, torch.float16])
def test_reindex_matches_oracle(cuda_device, vdt):
    print(f"case reindex {vdt}", flush=True)
    rng = np.random.default_rng(13)
    tc, ntiles = 8, 500
    cols = rng.integers(-1, 4000, ntiles * tc).astype(np.int32)
    cols[::17] = -1
    vals = rng.standard_normal(ntiles * 16 * tc).astype(np.float32)
    vals = torch.from_numpy(vals).to(vdt).float().numpy()  # representable in vdt
    for active in (np.unique(rng.integers(0, 250, 90)).astype(np.int32),
                   np.unique(np.concatenate([[0], rng.integers(1, 250, 60)])).astype(np.int32),
                   np.zeros(0, np.int32)):
        oc, ov = oracle.reindex_prune(cols, vals, active, 16, tc)
        dv = torch.from_numpy(vals).to(cuda_device).to(vdt)
        v0 = dv._version
        out = core.reindex_bcsr(torch.from_numpy(cols).to(cuda_device), dv,
                                torch.from_numpy(active).to(cuda_device), 16, tc)
        torch.cuda.synchronize()
        assert dv._version > v0, "the in-place prune must bump the version caches key on"
        np.testing.assert_array_equal(out.cpu().numpy(), oc)
        np.testing.assert_array_equal(dv.float().cpu().numpy(), ov)


@pytest.mark.parametrize("cfg", ["c3", "c4"])
def test_build_full_size_forward_and_transposed(cuda_device, cfg):
    """BASELINE configs c3 (windows of up to 8,246 edges) and c4 (667
    windows above 16,384 edges, built each by one work-group from global
    scratch) at full size: the device build equals the oracle's converter
    (oracle.csr_to_bcsr, pinned to the reference's compiled
    convert_wrapper.cpp in tests/test_oracle.py), and the transposed build
    equals the oracle's converter on A^T's CSR (the edges put in column
    order by a stable host sort)."""
    print(f"case {cfg} full-size build", flush=True)
    g = synth.config_graph(cfg, device=cuda_device)
    n = g.num_nodes
    rp, ci, va = g.row_ptr.cpu().numpy(), g.col_idx.cpu().numpy(), g.values.cpu().numpy()
    dw, dc, dv = builder.csr_to_bcsr_device(n, n, g.row_ptr, g.col_idx, g.values, tile_cols=16)
    ow, oc, ov = oracle.csr_to_bcsr(n, rp, ci, va, 16, 16)
    _eq_np(dw, ow)
    _eq_np(dc, oc)
    _eq_np(dv, ov)
    del dw, dc, dv, ow, oc, ov
    print(f"case {cfg} full-size transposed build", flush=True)
    tw, tc_, tv = builder.csr_to_bcsr_device(n, n, g.row_ptr, g.col_idx, g.values, tile_cols=16, transpose=True)
    order = np.argsort(ci, kind="stable")
    rows = np.repeat(np.arange(n, dtype=np.int32), np.diff(rp))[order]
    trp = np.zeros(n + 1, np.int64)
    trp[1:] = np.cumsum(np.bincount(ci, minlength=n))
    ew, ec, ev = oracle.csr_to_bcsr(n, trp, rows, va[order], 16, 16)
    del order
    _eq_np(tw, ew)
    _eq_np(tc_, ec)
    _eq_np(tv, ev)


def _eq_np(d, o, step=1 << 26):
    """A device array equal to an oracle array (values compared as float32:
    the oracle carries them in float64, exactly), in chunks."""
    assert d.numel() == o.size, (d.numel(), o.size)
    for i in range(0, o.size, step):
        a = d[i:i + step].cpu().numpy()
        b = o[i:i + step].astype(a.dtype) if o.dtype != a.dtype else o[i:i + step]
        if not np.array_equal(a, b):
            j = i + int(np.flatnonzero(a != b)[0])
            raise AssertionError(f"first difference at {j}: device {a[j - i]!r}, oracle {b[j - i]!r}")


def test_build_c2_full_size(cuda_device):
    """BASELINE config c2 through the device builder equals the oracle's
    converter and the host converter."""
    print("case c2 build", flush=True)
    g = synth.config_graph("c2")
    ow, oc, ov = _oracle_bcsr(g, 16)
    hw, hc, hv = _host(g, 16)
    dw, dc, dv = builder.csr_to_bcsr_device(g.num_nodes, g.num_nodes, g.row_ptr.to(cuda_device),
                                            g.col_idx.to(cuda_device), g.values.to(cuda_device),
                                            tile_cols=16)
    _eq(dw, ow)
    _eq(dc, oc)
    _eq(dv, ov)
    _eq(hw, ow)
    _eq(hc, oc)
    _eq(hv, ov)
