"""BCSR SpMM forward (H1) on the GPU against the float64 oracle.

Tolerance (north_star): |Y - Y_ref| <= rtol * (|A| |X|) elementwise, computed
in float64 on the same quantised inputs, with rtol = 1e-2 for float16 /
bfloat16 inputs and 1e-5 for float32.
"""
import numpy as np
import pytest
import torch

import oracle
from _fullsize import DT, assert_tight, rows_nnz_of
from graph_rws_amd import core, synth
from graph_rws_amd.data import BCSRGraph

pytestmark = pytest.mark.gpu

RTOL = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}


def _bcsr(g, tc, dev, vdt=torch.float32):
    win, cols, vals = core.csr_to_bcsr_cpu(g.num_nodes, g.row_ptr, g.col_idx, g.values, 16, tc)
    return BCSRGraph(g.num_nodes, g.nnz, 16, tc, win, cols, vals, device=dev,
                     num_cols=g.num_nodes, values_dtype=vdt)


def _check(G, X, Y, xdt):
    """Compare the device result with the oracle on the quantised inputs, in
    the contract tier (RTOL |A||X|) and the tight tier of tests/_fullsize.py
    (the arithmetic's own bound: one output rounding plus C k 2^-24 |A||X|)."""
    vq = G.values_condensed.to(xdt).double().cpu().numpy() if G.values_condensed.dtype != xdt \
        else G.values_condensed.double().cpu().numpy()
    win = G.window_offset.cpu().numpy()
    Yr, Ya = oracle.bcsr_spmm(win, G.original_col_indices.cpu().numpy(),
                              vq, 16, G.tile_cols, X.double().cpu().numpy())
    Yd = Y.double().cpu().numpy()
    err = np.abs(Yd - Yr)
    bound = RTOL[xdt] * Ya
    bad = err > bound
    assert not bad.any(), (f"{bad.sum()} of {bad.size} elements out of tolerance; "
                           f"worst excess {float((err - bound).max()):.3e}")
    dt = DT[xdt]
    assert_tight(Yd, Yr, Ya, rows_nnz_of(win, vq, G.tile_cols), dt, dt, DT[Y.dtype])
    return Yr


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("tc", [8, 16])
@pytest.mark.parametrize("N", [1, 7, 16, 17, 41, 64, 128, 200])
def test_spmm_parity_random(cuda_device, xdt, tc, N):
    print(f"case random xdt={xdt} tc={tc} N={N}", flush=True)
    g = synth.random_graph(333, 9.0, seed=N + tc)
    G = _bcsr(g, tc, cuda_device)
    X = synth.features(g.num_nodes, N, seed=N, device=cuda_device).to(xdt)
    Y = G.spmm(X)
    torch.cuda.synchronize()
    assert Y.shape == (16 * G.num_windows, N) and Y.dtype == xdt
    _check(G, X, Y, xdt)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("tc", [8, 16])
def test_spmm_parity_low_precision_values(cuda_device, xdt, tc):
    """values stored in the 16-bit type (no in-kernel conversion)."""
    print(f"case lowprec-values xdt={xdt} tc={tc}", flush=True)
    g = synth.random_graph(500, 12.0, seed=3)
    G = _bcsr(g, tc, cuda_device, vdt=xdt)
    X = synth.features(g.num_nodes, 96, seed=4, device=cuda_device).to(xdt)
    Y = G.spmm(X)
    torch.cuda.synchronize()
    _check(G, X, Y, xdt)


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16])
@pytest.mark.parametrize("slabs", [1, 2, 3, 16])
def test_spmm_split_windows(cuda_device, xdt, slabs):
    """Power-law graph with hub windows, forced splitting over work items."""
    print(f"case split xdt={xdt} slabs={slabs}", flush=True)
    g = synth.chung_lu(3000, 40000, 2.1, seed=11)
    G = _bcsr(g, 16, cuda_device)
    plan = core.build_spmm_plan(G.window_offset, G.num_tiles, 16, slabs)
    assert plan.num_split > 0
    X = synth.features(g.num_nodes, 80, seed=5, device=cuda_device).to(xdt)
    Y = core.spmm(G.window_offset, G.original_col_indices, G.values_condensed, X, 16, plan=plan)
    Y0 = core.spmm(G.window_offset, G.original_col_indices, G.values_condensed, X, 16, plan=None)
    torch.cuda.synchronize()
    _check(G, X, Y, xdt)
    _check(G, X, Y0, xdt)


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("slabs,N", [(2, 80), (3, 128), (16, 300)])
def test_plan_order_longest_first_same_results(cuda_device, xdt, slabs, N):
    """grws_spmm_plan_order (what build_spmm_plan applies when the plan
    splits windows): the items are a permutation of the window-order plan's,
    each eighth of the list (one XCD's share) keeps its own items, longest
    first, equal lengths in window order; the product (forward and over A^T)
    equals the window-order plan's bit for bit."""
    print(f"case plan order xdt={xdt} slabs={slabs} N={N}", flush=True)
    g = synth.chung_lu(3000, 40000, 2.1, seed=11)
    G = _bcsr(g, 16, cuda_device, vdt=xdt)
    p0 = core.build_spmm_plan(G.window_offset, G.num_tiles, 16, slabs, order=False)
    p1 = core.build_spmm_plan(G.window_offset, G.num_tiles, 16, slabs)
    assert p0.num_split > 0 and p1.num_items == p0.num_items and p1.num_slots == p0.num_slots
    n = p0.num_items
    i0 = p0.items.view(-1, 4)[:n].cpu().numpy()
    i1 = p1.items.view(-1, 4)[:n].cpu().numpy()
    per = (n + 7) // 8
    for k in range(8):
        a, b = i0[k * per:(k + 1) * per], i1[k * per:(k + 1) * per]
        la, lb = a[:, 2] - a[:, 1], b[:, 2] - b[:, 1]
        want = a[np.argsort(-la, kind="stable")]
        np.testing.assert_array_equal(b, want)
        assert (np.diff(lb) <= 0).all()
    ns = 3 * p0.num_split
    assert torch.equal(p1.split[:ns], p0.split[:ns])
    X = synth.features(g.num_nodes, N, seed=5, device=cuda_device).to(xdt)
    Y0 = core.spmm(G.window_offset, G.original_col_indices, G.values_condensed, X, 16, plan=p0)
    Y1 = core.spmm(G.window_offset, G.original_col_indices, G.values_condensed, X, 16, plan=p1)
    torch.cuda.synchronize()
    assert torch.equal(Y1.view(torch.uint8), Y0.view(torch.uint8))
    _check(G, X, Y1, xdt)


def test_plan_order_applies_to_split_plans_only(cuda_device):
    """build_spmm_plan orders the items when the plan splits windows (the
    hub windows of a power-law graph) and keeps window order otherwise (a
    graph whose windows all fit one item keeps its neighbours together)."""
    print("case plan order rule", flush=True)
    g = synth.chung_lu(3000, 40000, 2.1, seed=11)
    G = _bcsr(g, 16, cuda_device)
    big = core.build_spmm_plan(G.window_offset, G.num_tiles, 16, 1 << 20)
    assert big.num_split == 0
    n = big.num_items
    assert (np.diff(big.items.view(-1, 4)[:n, 0].cpu().numpy()) >= 0).all()  # window order kept
    split = core.build_spmm_plan(G.window_offset, G.num_tiles, 16, 2)
    ref = core.build_spmm_plan(G.window_offset, G.num_tiles, 16, 2, order=False)
    m = 4 * ref.num_items
    assert split.num_split > 0 and not torch.equal(split.items[:m], ref.items[:m])


def test_spmm_deterministic(cuda_device):
    print("case determinism", flush=True)
    g = synth.chung_lu(4000, 60000, 2.1, seed=12)
    G = _bcsr(g, 16, cuda_device)
    plan = core.build_spmm_plan(G.window_offset, G.num_tiles, 16, 2)
    X = synth.features(g.num_nodes, 128, seed=6, device=cuda_device).to(torch.float16)
    a = core.spmm(G.window_offset, G.original_col_indices, G.values_condensed, X, 16, plan=plan)
    b = core.spmm(G.window_offset, G.original_col_indices, G.values_condensed, X, 16, plan=plan)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_spmm_padding_never_reads_x(cuda_device):
    """NaN in every X row no column references must not reach Y: -1 slots and
    out-of-range columns are masked at the load."""
    print("case nan-poison", flush=True)
    n = 400
    rng = np.random.default_rng(7)
    rows = rng.integers(0, n, 3000)
    cols = rng.integers(0, n // 2, 3000)          # only the first half is referenced
    key = np.unique(rows * n + cols)
    rows, cols = key // n, key % n
    rp = np.zeros(n + 1, np.int64)
    np.add.at(rp, rows + 1, 1)
    rp = np.cumsum(rp)
    g = synth.CSRGraph(n, torch.from_numpy(rp), torch.from_numpy(cols.astype(np.int32)),
                       torch.from_numpy(rng.standard_normal(cols.size).astype(np.float32)))
    for tc in (8, 16):
        G = _bcsr(g, tc, cuda_device)
        X = synth.features(n, 48, seed=1, device=cuda_device)
        X[n // 2:] = float("nan")
        Y = G.spmm(X)
        torch.cuda.synchronize()
        assert torch.isfinite(Y).all()
        _check(G, X[: n // 2].contiguous(), Y, torch.float32)


def test_spmm_empty_windows_and_short_x(cuda_device):
    """Windows without tiles produce zero rows; columns >= x_rows contribute
    nothing (x shorter than num_cols)."""
    print("case empty-windows", flush=True)
    n = 100
    rp = np.zeros(n + 1, np.int64)
    rp[50:] = 3                                    # only row 49 has edges
    cols = np.array([2, 60, 99], np.int32)
    vals = np.array([1.0, 2.0, 4.0], np.float32)
    g = synth.CSRGraph(n, torch.from_numpy(rp), torch.from_numpy(cols), torch.from_numpy(vals))
    G = _bcsr(g, 8, cuda_device)
    X = torch.ones(70, 16, device=cuda_device)      # rows 70.. do not exist
    Y = G.spmm(X)
    torch.cuda.synchronize()
    expect = torch.zeros(112, 16)
    expect[49] = 3.0
    assert torch.equal(Y.cpu(), expect)


def test_spmm_tc_dropin_signature(cuda_device):
    """core.spmm_tc keeps the reference's (C, ms) return (bind.cpp:124-130)."""
    print("case spmm_tc", flush=True)
    g = synth.random_graph(257, 6.0, seed=21)
    G = _bcsr(g, 8, cuda_device)
    X = synth.features(g.num_nodes, 64, seed=2, device=cuda_device)
    C, ms = core.spmm_tc(G.window_offset, G.original_col_indices, G.values_condensed, X, 8)
    torch.cuda.synchronize()
    assert isinstance(ms, float) and C.shape == (16 * G.num_windows, 64)
    _check(G, X, C, torch.float32)


def test_spmm_c2_full_size(cuda_device):
    """BASELINE config c2 (169,343 nodes, ~2.33M nnz, N=128, f16 and bf16)."""
    print("case c2 full", flush=True)
    g = synth.config_graph("c2")
    G = _bcsr(g, 16, cuda_device)
    for xdt in (torch.float16, torch.bfloat16):
        X = synth.features(g.num_nodes, 128, seed=2, device=cuda_device).to(xdt)
        Y = G.spmm(X)
        torch.cuda.synchronize()
        _check(G, X, Y, xdt)


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16])
def test_spmm_ragged_width_row_padding(cuda_device, xdt):
    """A ragged width (41 columns) read from a wider buffer runs the vector
    kernel over the row padding: NaN in the padding columns must stay out of
    the first 41 output columns.  The explicit-out path (element loads) and
    the zero-padded copy path give the same values."""
    print(f"case ragged xdt={xdt}", flush=True)
    g = synth.chung_lu(2000, 30000, 2.1, seed=21)
    G = _bcsr(g, 16, cuda_device)
    buf = torch.full((g.num_nodes, 48), float("nan"), device=cuda_device, dtype=xdt)
    buf[:, :41] = synth.features(g.num_nodes, 41, seed=2, device=cuda_device).to(xdt)
    X = buf[:, :41]
    Y = G.spmm(X)
    Yc = G.spmm(X.contiguous())
    Yo = torch.empty(16 * G.num_windows, 41, device=cuda_device, dtype=xdt)
    G.spmm(X, out=Yo)
    torch.cuda.synchronize()
    assert Y.shape == (16 * G.num_windows, 41) and bool(torch.isfinite(Y).all())
    _check(G, X.contiguous(), Y, xdt)
    _check(G, X.contiguous(), Yo, xdt)
    assert torch.equal(Y, Yc)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N", [300, 608, 520])
@pytest.mark.parametrize("slabs", [None, 2])
def test_spmm_wide_split_launches(cuda_device, xdt, N, slabs):
    """Widths above 256 that are not multiples of it run as 256-column
    chunks plus a narrower launch for the rest (and, with split windows,
    two partial fixups at different column offsets)."""
    print(f"case wide xdt={xdt} N={N} slabs={slabs}", flush=True)
    g = synth.chung_lu(2500, 40000, 2.1, seed=N)
    G = _bcsr(g, 16, cuda_device, vdt=xdt)
    X = synth.features(g.num_nodes, N, seed=N + 1, device=cuda_device).to(xdt)
    if slabs is None:
        Y = G.spmm(X)
    else:
        plan = core.build_spmm_plan(G.window_offset, G.num_tiles, 16, slabs)
        assert plan.num_split > 0
        Y = core.spmm(G.window_offset, G.original_col_indices, G.values_condensed, X, 16, plan=plan)
    torch.cuda.synchronize()
    _check(G, X, Y, xdt)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_gather_input_aligned_copy(cuda_device, xdt):
    """A graph that gathers each row many times multiplies X through a copy
    whose rows start on 128-byte lines when X's pitch is not a multiple of
    128 bytes (112 columns here): same bits as the product on X itself, the
    copy is kept while X is alive and unmodified, and redone after an
    in-place change."""
    print(f"case aligned-copy xdt={xdt}", flush=True)
    g = synth.chung_lu(3000, 200000, 2.1, seed=4)
    G = _bcsr(g, 16, cuda_device, vdt=xdt)
    assert G.num_tiles * 16 >= 8 * g.num_nodes
    X = synth.features(g.num_nodes, 112, seed=8, device=cuda_device).to(xdt)
    assert X.stride(0) * X.element_size() % 128 != 0
    args = (G.window_offset, G.original_col_indices, G.values_condensed)
    ref = core.spmm(*args, X, 16, plan=G.spmm_plan(112))       # the kernel on the 224-byte pitch
    Y = G.spmm(X)
    xa = G._cache["aligned_x"][id(X)][2]
    assert xa.stride(0) * xa.element_size() % 128 == 0 and torch.equal(xa, X)
    # another, short-lived input in between (a later layer's product on the
    # same graph): it gets its own copy, dropped with it, and X's stays
    T = synth.features(g.num_nodes, 47, seed=9, device=cuda_device).to(xdt)
    refT = core.spmm(*args, T, 16, plan=G.spmm_plan(47))
    YT = G.spmm(T)
    assert id(T) in G._cache["aligned_x"]
    torch.cuda.synchronize()
    assert torch.equal(YT.view(torch.int16), refT.view(torch.int16))
    tid = id(T)
    del T
    assert tid not in G._cache["aligned_x"]
    Y2 = G.spmm(X)
    assert G._cache["aligned_x"][id(X)][2] is xa                # reused
    torch.cuda.synchronize()
    assert torch.equal(Y.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(Y2.view(torch.int16), ref.view(torch.int16))
    with torch.no_grad():
        X.mul_(2)
    Y3 = G.spmm(X)
    assert G._cache["aligned_x"][id(X)][2] is not xa
    ref3 = core.spmm(*args, X, 16, plan=G.spmm_plan(112))
    torch.cuda.synchronize()
    assert torch.equal(Y3.view(torch.int16), ref3.view(torch.int16))


def test_ragged_width_copy_is_line_aligned(cuda_device):
    """A ragged width widened by copy gets 128-byte row pitch (41 -> 48
    columns at a 64-element pitch)."""
    from graph_rws_amd.core.ops import _widen
    x = torch.randn(1000, 41, device=cuda_device).half()
    w = _widen(x, 8)
    assert w.shape == (1000, 48) and w.stride(0) == 64
    assert torch.equal(w[:, :41], x) and not bool(w[:, 41:].any())


@pytest.mark.parametrize("tc", [8, 16])
@pytest.mark.parametrize("N", [4, 16, 64, 128, 200])
@pytest.mark.parametrize("slabs", [None, 2])
def test_fp32_buffer_kernel_equals_element_masked(cuda_device, tc, N, slabs):
    """fp32 X runs the buffer-load kernel (v_mfma_f32_16x16x4f32, the same
    MFMA sequence as the element-masked kernel): the same bits as the
    element-masked kernel, forced with the GRWS_SPMM_KERNEL=1 override."""
    print(f"case fp32 buf tc={tc} N={N} slabs={slabs}", flush=True)
    g = synth.chung_lu(2500, 30000, 2.1, seed=N + tc)
    G = _bcsr(g, tc, cuda_device)
    plan = None if slabs is None else core.build_spmm_plan(G.window_offset, G.num_tiles, tc, slabs)
    X = synth.features(g.num_nodes, N, seed=N, device=cuda_device)
    args = (G.window_offset, G.original_col_indices, G.values_condensed, X, tc)
    Yb = core.spmm(*args, plan=plan)
    from graph_rws_amd.core.ops import spmm_tuning
    with spmm_tuning(GRWS_SPMM_KERNEL=1):
        Ye = core.spmm(*args, plan=plan)
        torch.cuda.synchronize()
    assert torch.equal(Yb.view(torch.int32), Ye.view(torch.int32))
    _check(G, X, Yb, torch.float32)


def _with_env(env, fn):
    """fn() under the SpMM tuning overrides env (name -> value)."""
    from graph_rws_amd.core.ops import spmm_tuning
    with spmm_tuning(**{k: int(v) for k, v in env.items()}):
        return fn()


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("slabs", [None, 3])
@pytest.mark.parametrize("big_x", [False, True])
def test_chunk_widths_and_work_orders_agree(cuda_device, xdt, slabs, big_x):
    """The chunk width (16..256 columns per work-group) and the work order
    (chunk-major or per-XCD shares of the (chunk, window) pairs) change only
    which work-group computes an output column, not the order of its sum:
    every variant gives the same bits.  big_x: X has 600k rows, past the
    256 MB a 256-column slice may take before the library picks 128-column
    chunks by itself."""
    print(f"case chunk-orders xdt={xdt} slabs={slabs} big_x={big_x}", flush=True)
    g = synth.chung_lu(3000, 50000, 2.1, seed=11)
    G = _bcsr(g, 16, cuda_device, vdt=xdt)
    N = 512
    rows = 600_000 if big_x else g.num_nodes
    X = synth.features(rows, N, seed=12, device=cuda_device).to(xdt)
    plan = None if slabs is None else core.build_spmm_plan(G.window_offset, G.num_tiles, 16, slabs)
    args = (G.window_offset, G.original_col_indices, G.values_condensed, X, 16)
    ref = core.spmm(*args, plan=plan)
    torch.cuda.synchronize()
    for env in ({"GRWS_SPMM_ORDER": "0"}, {"GRWS_SPMM_NBLK": "8", "GRWS_SPMM_ORDER": "0"},
                {"GRWS_SPMM_NBLK": "8", "GRWS_SPMM_ORDER": "1"}, {"GRWS_SPMM_NBLK": "16", "GRWS_SPMM_ORDER": "1"},
                {"GRWS_SPMM_NBLK": "2", "GRWS_SPMM_ORDER": "1"}):
        Y = _with_env(env, lambda: core.spmm(*args, plan=plan))
        torch.cuda.synchronize()
        assert torch.equal(Y.view(torch.int16), ref.view(torch.int16)), env
    _check(G, X[: g.num_nodes], ref, xdt)


_RESIDUAL_CASES = [(xdt, v) for xdt in (torch.float32, torch.float16, torch.bfloat16)
                   for v in ("plain", "split", "packed", "two_waves", "element_masked")
                   if not (v == "packed" and xdt == torch.float32)]  # packed tiles hold 16-bit values


@pytest.mark.parametrize("xdt,variant", _RESIDUAL_CASES)
@pytest.mark.parametrize("N", [16, 47, 128, 256, 300])
def test_spmm_residual_parity(cuda_device, xdt, variant, N):
    """Y = A X + R on the first r_rows rows (grws_spmm_residual): against the
    float64 oracle plus R, with the oracle's bound widened by |R| for the
    one rounding of the sum; rows past r_rows equal the plain product."""
    import os
    print(f"case residual xdt={xdt} N={N} {variant}", flush=True)
    g = synth.chung_lu(2500, 40000, 2.1, seed=N + 3)
    G = _bcsr(g, 16, cuda_device, vdt=torch.float32 if xdt == torch.float32 else xdt)
    X = synth.features(g.num_nodes, N, seed=N, device=cuda_device).to(xdt)
    rows = 16 * G.num_windows
    r_rows = rows - 37
    R = (synth.features(r_rows, N, seed=N + 9, device=cuda_device) * 4).to(xdt)
    args = (G.window_offset, G.original_col_indices, G.values_condensed, X, 16)
    plan = core.build_spmm_plan(G.window_offset, G.num_tiles, 16, 2) if variant == "split" else None
    packed = core.pack_tiles(G.window_offset, G.original_col_indices, G.values_condensed, 16) \
        if variant == "packed" else None
    env = {"two_waves": {"GRWS_SPMM_WAVES": "2"}, "element_masked": {"GRWS_SPMM_KERNEL": "1"}}.get(variant, {})
    from graph_rws_amd.core.ops import spmm_tuning
    with spmm_tuning(**{k: int(v) for k, v in env.items()}):
        Y = core.spmm(*args, plan=plan, packed=packed, residual=R)
        Y0 = core.spmm(*args, plan=plan, packed=packed)
        torch.cuda.synchronize()
    vq = G.values_condensed.double().cpu().numpy()
    Yr, Ya = oracle.bcsr_spmm(G.window_offset.cpu().numpy(), G.original_col_indices.cpu().numpy(), vq, 16, 16,
                              X.double().cpu().numpy())
    Rn = R.double().cpu().numpy()
    Yr[:r_rows] += Rn
    Ya[:r_rows] += np.abs(Rn)
    err = np.abs(Y.double().cpu().numpy() - Yr)
    assert (err <= RTOL[xdt] * Ya).all()
    # tight tier: the residual is one more term of its rows' sums
    k = rows_nnz_of(G.window_offset.cpu().numpy(), vq, 16)
    k[:r_rows] += 1
    dt = DT[xdt]
    assert_tight(Y.double().cpu().numpy(), Yr, Ya, k, DT[G.values_condensed.dtype], dt, dt)
    assert torch.equal(Y[r_rows:], Y0[r_rows:])


def test_spmm_residual_in_place(cuda_device):
    """R may be the output itself: Y = A X + Y."""
    print("case residual in place", flush=True)
    g = synth.chung_lu(2000, 30000, 2.1, seed=5)
    G = _bcsr(g, 16, cuda_device, vdt=torch.float16)
    X = synth.features(g.num_nodes, 64, seed=6, device=cuda_device).half()
    args = (G.window_offset, G.original_col_indices, G.values_condensed, X, 16)
    Y = synth.features(16 * G.num_windows, 64, seed=7, device=cuda_device).half()
    R = Y.clone()
    ref = core.spmm(*args, residual=R)
    core.spmm(*args, out=Y, residual=Y)
    torch.cuda.synchronize()
    assert torch.equal(Y.view(torch.int16), ref.view(torch.int16))
