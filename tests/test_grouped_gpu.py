"""Grouped tiles (grws_group_tiles_count/_fill, grws_spmm_grouped).

Checks:
  * the layout the device writes restates A exactly: decoding it with numpy
    (the format declared in include/grws.h: per group the union columns in
    ascending order, 16 per slab, -1 after the last; per slab and window a
    packed 16x16 sub-tile) gives back the dense matrix of the BCSR graph,
    bit for bit, for group sizes 2, 4 and 8 and tiles of 16 and 8 columns;
  * the SpMM over grouped tiles meets the float64 oracle's tolerance
    (|Y - Y_ref| <= 1e-2 |A| |X| for 16-bit inputs) on every kernel shape
    (windows per wave 1, 2, 4; waves per group 1, 2, 4; 128-, 256- and
    320-column chunks and the narrower last launch), with the residual, and
    on a partial last group; it stays within one rounding of the output
    dtype of the window-by-window kernel;
  * 4-window groups multiply slab pairs on the 16x16x32 MFMA by default:
    against the oracle and the 16x16x16 kernel, with groups of odd slab
    counts (half a pair at the end).
"""

import numpy as np
import pytest
import torch

import oracle
from _fullsize import DT, assert_tight, rows_nnz_of
from graph_rws_amd import core, synth
from graph_rws_amd.core import ops
from graph_rws_amd.data import BCSRGraph

pytestmark = pytest.mark.gpu


def _graph(dev, vdt, tc, scale=0.004, cfg="c3"):
    g = synth.config_graph(cfg, scale=scale)
    win, cols, vals = core.csr_to_bcsr_cpu(g.num_nodes, g.row_ptr, g.col_idx, g.values, 16, tc)
    return g, BCSRGraph(g.num_nodes, g.nnz, 16, tc, win, cols, vals, device=dev, num_cols=g.num_nodes,
                        values_dtype=vdt)


def _dense_from_bcsr(G):
    win = G.window_offset.cpu().numpy()
    cols = G.original_col_indices.cpu().numpy().reshape(-1, G.tile_cols)
    bits = G.values_condensed.view(torch.int16).cpu().numpy().astype(np.uint16).reshape(-1, 16, G.tile_cols)
    D = np.zeros((16 * G.num_windows, G.num_cols), np.uint16)
    for w in range(G.num_windows):
        for t in range(win[w], win[w + 1]):
            for c in range(G.tile_cols):
                col = cols[t, c]
                if 0 <= col < G.num_cols:
                    D[16 * w:16 * w + 16, col] = bits[t, :, c]
    return D


def _dense_from_grouped(gt, W, num_cols):
    goff = gt.group_offset.cpu().numpy()
    gcols = gt.col_indices.cpu().numpy().reshape(-1, 16)
    hdr = gt.header.cpu().numpy().view(np.uint32).reshape(-1, gt.group_size, 4, 3)
    vals = gt.values.view(torch.int16).cpu().numpy().astype(np.uint16)
    G = gt.group_size
    D = np.zeros((16 * W, num_cols), np.uint16)
    seen = 0
    for q in range(gt.num_groups):
        c = gcols[goff[q]:goff[q + 1]].reshape(-1)
        valid = c[c >= 0]
        assert (np.diff(valid) > 0).all(), f"group {q}: union columns not ascending"
        assert (c[len(valid):] == -1).all(), f"group {q}: padding not at the end"
        assert len(c) - len(valid) < 16
        for s in range(goff[q], goff[q + 1]):
            for wi in range(G):
                for g in range(4):
                    lo, hi, start = hdr[s, wi, g]
                    m = int(lo) | (int(hi) << 32)
                    k = 0
                    for bit in range(64):
                        if (m >> bit) & 1:
                            r = 4 * g + bit // 16
                            col = gcols[s, bit % 16]
                            assert col >= 0, "a value in a padding column"
                            row = 16 * (q * G + wi) + r
                            assert row < 16 * W
                            D[row, col] = vals[start + k]
                            k += 1
                            seen += 1
    assert seen == gt.num_values
    return D


@pytest.mark.parametrize("G,tc,vdt", [(4, 16, torch.float16), (2, 16, torch.bfloat16), (8, 16, torch.float16),
                                      (4, 8, torch.bfloat16)])
def test_grouped_layout_restates_a(cuda_device, G, tc, vdt):
    print(f"case grouped layout G={G} tc={tc} {vdt}", flush=True)
    g, A = _graph(cuda_device, vdt, tc, scale=0.002)
    gt = ops.group_tiles(A.window_offset, A.original_col_indices, A.values_condensed, tc, A.num_cols,
                         group_size=G, max_ratio=1.0, max_skew=1e9)
    assert gt is not None and gt.num_groups == (A.num_windows + G - 1) // G
    np.testing.assert_array_equal(_dense_from_grouped(gt, A.num_windows, A.num_cols), _dense_from_bcsr(A))
    # community structure: the union is smaller than the windows' own slots
    assert gt.slot_ratio < 0.9


@pytest.mark.parametrize("G", [2, 4])
def test_grouped_union_bitmap_matches_sort(cuda_device, G):
    """Graphs of at most 2^18 columns build their groups' unions from LDS
    bitmaps, wider ones by a sort: the same layout bit for bit.  The columns
    are shifted to end at 2^18 - 1 (the bitmap's last bit), then the same
    arrays are declared 2^18 + 1 columns wide (the sort)."""
    print(f"case grouped union bitmap vs sort G={G}", flush=True)
    g, A = _graph(cuda_device, torch.float16, 16, scale=0.002)
    shift = (1 << 18) - A.num_cols
    cols = A.original_col_indices.clone()
    cols[cols >= 0] += shift
    a = ops.group_tiles(A.window_offset, cols, A.values_condensed, 16, 1 << 18, group_size=G,
                        max_ratio=1.0, max_skew=1e9)
    b = ops.group_tiles(A.window_offset, cols, A.values_condensed, 16, (1 << 18) + 1, group_size=G,
                        max_ratio=1.0, max_skew=1e9)
    assert a is not None and b is not None
    for name in ("group_offset", "col_indices", "header", "values"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    Da = _dense_from_grouped(a, A.num_windows, 1 << 18)
    np.testing.assert_array_equal(Da[:, shift:], _dense_from_bcsr(A))
    assert not Da[:, :shift].any()


def _oracle_check(A, X, Y, R=None):
    """The float64 oracle (residual R added to its rows), in the contract
    tier (1e-2 |A||X|) and the tight tier of tests/_fullsize.py."""
    vq = A.values_condensed.double().cpu().numpy()
    win = A.window_offset.cpu().numpy()
    Yr, Ya = oracle.bcsr_spmm(win, A.original_col_indices.cpu().numpy(), vq, 16,
                              A.tile_cols, X.double().cpu().numpy())
    k = rows_nnz_of(win, vq, A.tile_cols)
    if R is not None:
        Rn = R.double().cpu().numpy()
        Yr[:Rn.shape[0]] += Rn
        Ya[:Rn.shape[0]] += np.abs(Rn)
        k[:Rn.shape[0]] += 1
    Yd = Y.double().cpu().numpy()
    err = np.abs(Yd - Yr)
    bad = err > 1e-2 * Ya
    assert not bad.any(), f"{bad.sum()} of {bad.size} out of tolerance; worst {float((err - 1e-2 * Ya).max()):.3e}"
    dt = DT[X.dtype]
    assert_tight(Yd, Yr, Ya, k, DT[A.values_condensed.dtype], dt, DT[Y.dtype])


SHAPES = [  # (group size, windows per wave, column blocks of the first launch;
    # 16 at N = 608 runs 320-column chunks, with padded gathers at 4 waves)
    (4, 2, 16), (4, 1, 16), (4, 4, 8), (4, 2, 8), (2, 2, 16), (2, 1, 16), (2, 2, 8), (8, 2, 16), (8, 4, 8),
    (8, 2, 8)]


@pytest.mark.parametrize("G,wpw,nblk", SHAPES)
@pytest.mark.parametrize("N", [608, 256, 96, 48])
def test_grouped_spmm_meets_oracle(cuda_device, monkeypatch, G, wpw, nblk, N):
    print(f"case grouped spmm G={G} wpw={wpw} nblk={nblk} N={N}", flush=True)
    monkeypatch.setattr(ops, "GROUP_MIN_N", 0)  # the grouped kernel at every width
    _, A = _graph(cuda_device, torch.float16, 16, scale=0.004)
    gt = ops.group_tiles(A.window_offset, A.original_col_indices, A.values_condensed, 16, A.num_cols,
                         group_size=G, max_ratio=1.0, max_skew=1e9)
    assert gt is not None
    torch.manual_seed(N + G)
    X = torch.randn(A.num_cols, N, device=cuda_device).half()
    with ops.spmm_tuning(GRWS_GRP_WPW=wpw, GRWS_GRP_NBLK=nblk):
        Y = ops.spmm(A.window_offset, A.original_col_indices, A.values_condensed, X, 16, grouped=gt)
        torch.cuda.synchronize()
    _oracle_check(A, X, Y)
    Yw = ops.spmm(A.window_offset, A.original_col_indices, A.values_condensed, X, 16)
    # one rounding of fp16 apart at most: the sums differ only in fp32 order
    torch.testing.assert_close(Y.float(), Yw.float(), rtol=2 ** -10, atol=2 ** -14)


@pytest.mark.parametrize("vdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N", [608, 256, 96, 48])
@pytest.mark.parametrize("cfg,scale,tc", [("c3", 0.004, 16), ("c4", 0.002, 16), ("c3", 0.004, 8)])
def test_grouped_slab_pairs_match_single_slabs(cuda_device, monkeypatch, vdt, N, cfg, scale, tc):
    """4-window groups run slab pairs on the 16x16x32 MFMA by default
    (spmm_grp2_kernel; GRWS_GRP_K32=0 selects the 16x16x16 kernel): both
    meet the oracle in both tiers and stay within one output rounding of
    each other (the same exact sums in another fp32 order).  A group of an
    odd slab count ends with half a pair: the small c3-shaped graph is
    nearly dense (every group 59 slabs), the sparse c4-shaped one has
    groups of both parities.  The grouped layout is the same whether the
    graph's tiles are 16 or 8 columns wide (the reference's default)."""
    print(f"case grouped slab pairs {cfg} tc={tc} {vdt} N={N}", flush=True)
    monkeypatch.setattr(ops, "GROUP_MIN_N", 0)
    _, A = _graph(cuda_device, vdt, tc, scale=scale, cfg=cfg)
    gt = ops.group_tiles(A.window_offset, A.original_col_indices, A.values_condensed, tc, A.num_cols,
                         group_size=4, max_ratio=10.0, max_skew=1e9)
    slabs = (gt.group_offset[1:] - gt.group_offset[:-1]).cpu()
    assert bool((slabs % 2 == 1).any())
    if cfg == "c4":
        assert bool((slabs % 2 == 0).any())
    torch.manual_seed(N + 17)
    X = torch.randn(A.num_cols, N, device=cuda_device).to(vdt)
    assert int(ops.L.load().grws_spmm_get_tuning(b"GRWS_GRP_K32")) == -1  # the default: slab pairs
    Y2 = ops.spmm(A.window_offset, A.original_col_indices, A.values_condensed, X, tc, grouped=gt)
    with ops.spmm_tuning(GRWS_GRP_K32=0):
        Y1 = ops.spmm(A.window_offset, A.original_col_indices, A.values_condensed, X, tc, grouped=gt)
    torch.cuda.synchronize()
    _oracle_check(A, X, Y2)
    _oracle_check(A, X, Y1)
    u = 2 ** -10 if vdt == torch.float16 else 2 ** -7
    torch.testing.assert_close(Y2.float(), Y1.float(), rtol=u, atol=2 ** -14)


@pytest.mark.parametrize("vdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N,pad", [(608, 640), (576, 576), (320, 320), (384, 384), (256, 256), (200, 200),
                                   (96, 104)])
@pytest.mark.parametrize("cfg,scale", [("c3", 0.004), ("c4", 0.002)])
def test_slab_pairs_direct_loads_equal_register_staging(cuda_device, monkeypatch, vdt, N, pad, cfg, scale):
    """The slab-pair kernel stages X by direct loads into LDS by default
    (spmm_grp2d_kernel; GRWS_GRP_DMA=0 selects spmm_grp2_kernel, which stages
    through registers): the same sums in the same order, so the outputs are
    equal bit for bit, on every chunk width (320-column chunks, 256 plus a
    narrower tail, 128), with a row pitch wider than N, and twice in a row
    (the direct loads of one pair must land before any wave reads them)."""
    print(f"case slab pairs direct loads {cfg} {vdt} N={N} pitch={pad}", flush=True)
    monkeypatch.setattr(ops, "GROUP_MIN_N", 0)
    _, A = _graph(cuda_device, vdt, 16, scale=scale, cfg=cfg)
    gt = ops.group_tiles(A.window_offset, A.original_col_indices, A.values_condensed, 16, A.num_cols,
                         group_size=4, max_ratio=10.0, max_skew=1e9)
    torch.manual_seed(N + 29)
    X = torch.zeros(A.num_cols, pad, device=cuda_device, dtype=vdt)
    X[:, :N] = torch.randn(A.num_cols, N, device=cuda_device).to(vdt)
    X = X[:, :N]
    assert int(ops.L.load().grws_spmm_get_tuning(b"GRWS_GRP_DMA")) == -1  # the default: direct loads
    Yd = [ops.spmm(A.window_offset, A.original_col_indices, A.values_condensed, X, 16, grouped=gt)
          for _ in range(2)]
    with ops.spmm_tuning(GRWS_GRP_DMA=0):
        Yr = ops.spmm(A.window_offset, A.original_col_indices, A.values_condensed, X, 16, grouped=gt)
    torch.cuda.synchronize()
    for Y in Yd:
        assert torch.equal(Y.view(torch.int16), Yr.view(torch.int16))
    _oracle_check(A, X, Yd[0])


@pytest.mark.parametrize("vdt", [torch.float16, torch.bfloat16])
def test_grouped_spmm_residual_and_partial_group(cuda_device, monkeypatch, vdt):
    """Y = A X + R with R on a prefix of the rows; a window count that leaves
    the last group partial (its missing windows write nothing)."""
    print(f"case grouped residual {vdt}", flush=True)
    monkeypatch.setattr(ops, "GROUP_MIN_N", 0)
    _, A = _graph(cuda_device, vdt, 16, scale=0.003)
    gt = ops.group_tiles(A.window_offset, A.original_col_indices, A.values_condensed, 16, A.num_cols,
                         group_size=4, max_ratio=1.0, max_skew=1e9)
    torch.manual_seed(3)
    X = torch.randn(A.num_cols, 256, device=cuda_device).to(vdt)
    R = torch.randn(A.num_cols - 5, 256, device=cuda_device).to(vdt)
    Y = ops.spmm(A.window_offset, A.original_col_indices, A.values_condensed, X, 16, residual=R, grouped=gt)
    _oracle_check(A, X, Y, R)
    # a graph whose window count is not a multiple of the group size
    W = A.num_windows - (A.num_windows % 4) - 1
    T = int(A.window_offset[W])
    B = BCSRGraph(16 * W, 0, 16, 16, A.window_offset[:W + 1].clone(), A.original_col_indices[:T * 16].clone(),
                  A.values_condensed[:T * 256].clone(), device=cuda_device, num_rows=16 * W, num_cols=A.num_cols,
                  values_dtype=vdt)
    gb = ops.group_tiles(B.window_offset, B.original_col_indices, B.values_condensed, 16, B.num_cols,
                         group_size=4, max_ratio=1.0, max_skew=1e9)
    assert gb.num_groups == (W + 3) // 4 and W % 4 == 3
    Yb = ops.spmm(B.window_offset, B.original_col_indices, B.values_condensed, X, 16, grouped=gb)
    assert Yb.shape[0] == 16 * W
    _oracle_check(B, X, Yb)


def test_graph_groups_its_tiles_when_it_pays(cuda_device, monkeypatch):
    """BCSRGraph.spmm builds grouped tiles on the second product of a graph
    with community structure and uses them; a Chung-Lu graph (no community
    structure) is left on the window-by-window path."""
    print("case graph grouping policy", flush=True)
    _, A = _graph(cuda_device, torch.float16, 16, scale=0.01)
    X = torch.randn(A.num_cols, 256, device=cuda_device).half()
    y1 = A.spmm(X)
    y2 = A.spmm(X)
    gt = A._cache[("grouped", 4)][2]
    assert gt, "c3-like graph not grouped"
    assert gt.slot_ratio <= ops.GROUP_MAX_RATIO
    assert gt.group_size == ops.group_size_for(256) == 4  # the group size suits the product's width
    torch.testing.assert_close(y1.float(), y2.float(), rtol=2 ** -10, atol=2 ** -14)
    _oracle_check(A, X, y2)
    assert ops.group_size_for(608) == 4
    # one cached layout per group size, not the first width's: under a
    # policy that picks 2 windows above 256 columns, a graph first
    # multiplied 608 columns wide still gets 4-window tiles at 256 columns
    monkeypatch.setattr(ops, "group_size_for", lambda n: 2 if n > 256 else 4)
    _, A2 = _graph(cuda_device, torch.float16, 16, scale=0.01)
    X6 = torch.randn(A2.num_cols, 608, device=cuda_device).half()
    A2.spmm(X6)
    y6 = A2.spmm(X6)
    assert A2._cache[("grouped", 2)][2].group_size == 2
    _oracle_check(A2, X6, y6)
    X2 = torch.randn(A2.num_cols, 256, device=cuda_device).half()
    A2.spmm(X2)
    y2b = A2.spmm(X2)
    assert A2._cache[("grouped", 4)][2].group_size == 4
    assert A2._cache[("grouped", 2)][2].group_size == 2
    _oracle_check(A2, X2, y2b)
    _, B = _graph(cuda_device, torch.float16, 16, scale=0.01, cfg="c4")
    Xb = torch.randn(B.num_cols, 256, device=cuda_device).half()
    B.spmm(Xb)
    B.spmm(Xb)
    assert B._cache[("grouped", 4)][2] is False


@pytest.mark.parametrize("G", [2, 4])
def test_grouped_layout_special_values_and_empty_windows(cuda_device, G):
    """Windows with 0..40 tiles (a whole group may be empty), explicit zeros
    (dropped), -0.0, NaN and infinities (kept: nonzero bit patterns), -1
    padding: the grouped layout still decodes to the dense matrix bit for
    bit, and on the finite values the product meets the oracle."""
    from test_packed_gpu import _special_graph
    print(f"case grouped special G={G}", flush=True)
    A = _special_graph(cuda_device, torch.float16, seed=7)
    gt = ops.group_tiles(A.window_offset, A.original_col_indices, A.values_condensed, 16, A.num_cols,
                         group_size=G, max_ratio=10.0, max_skew=1e9)
    assert gt is not None
    np.testing.assert_array_equal(_dense_from_grouped(gt, A.num_windows, A.num_cols), _dense_from_bcsr(A))
    v = A.values_condensed.clone()
    v[~torch.isfinite(v)] = 0
    F = BCSRGraph(A.num_cols, 0, 16, 16, A.window_offset, A.original_col_indices, v, device=cuda_device,
                  num_cols=A.num_cols, values_dtype=torch.float16)
    gf = ops.group_tiles(F.window_offset, F.original_col_indices, F.values_condensed, 16, F.num_cols,
                         group_size=G, max_ratio=10.0, max_skew=1e9)
    torch.manual_seed(11)
    X = torch.randn(F.num_cols, 256, device=cuda_device).half()
    Y = ops.spmm(F.window_offset, F.original_col_indices, F.values_condensed, X, 16, grouped=gf)
    _oracle_check(F, X, Y)
