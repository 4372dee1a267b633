"""Packed tiles (grws_pack_tiles_count/_fill, grws_spmm_packed).

Two checks:
  * the layout the device writes equals a numpy restatement of the format
    declared in include/grws.h (per tile and row group q: a 64-bit mask with
    bit (r%4)*16 + c set for every slot whose value bits are not zero, the
    index of the group's first value, and the nonzero values in tile-then-slot
    order);
  * the SpMM over packed tiles is bit-identical to the SpMM over the dense
    tiles on every kernel shape (column blocks 1..16, one and two waves, the
    256-column split launches, split windows with their fixup), including
    -0.0, NaN and infinite values, explicitly stored zeros, full and empty
    tiles.  The dense SpMM is itself checked against the float64 oracle in
    test_spmm_gpu.py, and one case here repeats that check for the packed
    path.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from graph_rws_amd import core, synth
from graph_rws_amd.core import _lib as L
from graph_rws_amd.data import BCSRGraph

pytestmark = pytest.mark.gpu


def _pack_numpy(vals16: np.ndarray):
    """vals16: [T, 256] uint16 bit patterns -> (header [T, 4, 3] uint32, values uint16)."""
    nz = vals16 != 0
    counts = nz.sum(1)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.int64)
    T = vals16.shape[0]
    header = np.zeros((T, 4, 3), np.uint32)
    weights = (np.uint64(1) << np.arange(64, dtype=np.uint64))
    for q in range(4):
        grp = nz[:, 64 * q:64 * q + 64].astype(np.uint64)
        mask = (grp * weights).sum(1, dtype=np.uint64)
        header[:, q, 0] = (mask & np.uint64(0xFFFFFFFF)).astype(np.uint32)
        header[:, q, 1] = (mask >> np.uint64(32)).astype(np.uint32)
        header[:, q, 2] = (starts + nz[:, :64 * q].sum(1)).astype(np.uint32)
    return header, vals16[nz]


def _special_graph(dev, dt, seed=0):
    """Windows with 0..40 tiles of 16x16, densities 0, 0.02, 0.1, 0.5 and
    1.0 per tile, explicit zeros, -0.0, NaN and inf among the values, -1
    column padding in the last tile of a window."""
    rng = np.random.default_rng(seed)
    n = 4000
    W = 60
    ntiles = rng.integers(0, 41, W)
    ntiles[3] = 0
    win = np.concatenate([[0], np.cumsum(ntiles)]).astype(np.int64)
    T = int(win[-1])
    cols = np.full((T, 16), -1, np.int32)
    for w in range(W):
        k = int(ntiles[w]) * 16 - int(rng.integers(0, 16)) if ntiles[w] else 0
        c = np.sort(rng.choice(n, size=k, replace=False)).astype(np.int32)
        flat = np.full(int(ntiles[w]) * 16, -1, np.int32)
        flat[:k] = c
        cols[win[w]:win[w + 1]] = flat.reshape(-1, 16)
    last = int(np.nonzero(ntiles)[0][-1])
    cols[win[last + 1] - 1] = np.arange(n - 16, n, dtype=np.int32)   # last tile: real columns in every slot
    dens = rng.choice([0.0, 0.02, 0.1, 0.5, 1.0], size=T)
    dens[-1] = 0.3                                 # values up to the end of the packed array
    vals = rng.standard_normal((T, 256)).astype(np.float32)
    vals *= rng.random((T, 256)) < dens[:, None]
    vals = torch.from_numpy(vals).to(dt)
    bits = vals.view(torch.int16)
    flat = bits.view(-1)
    m = flat.numel()
    if m:
        idx = torch.from_numpy(rng.integers(0, m, 40))
        flat[idx[:10]] = -32768                      # -0.0
        specials = torch.tensor([float("nan"), float("inf"), -float("inf")], dtype=dt).view(torch.int16)
        flat[idx[10:20]] = specials[0]
        flat[idx[20:30]] = specials[1]
        flat[idx[30:]] = specials[2]
    G = BCSRGraph(n, 0, 16, 16, torch.from_numpy(win), torch.from_numpy(cols.reshape(-1)), vals.view(-1),
                  device=dev, num_cols=n, values_dtype=dt)
    return G


def _bits(t):
    return t.view(torch.int16)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_pack_layout_matches_restatement(cuda_device, dt):
    print(f"case pack-layout {dt}", flush=True)
    G = _special_graph(cuda_device, dt, seed=1)
    P = core.pack_tiles(G.window_offset, G.original_col_indices, G.values_condensed, 16)
    torch.cuda.synchronize()
    assert P is not None
    v16 = G.values_condensed.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1, 256)
    hdr, pv = _pack_numpy(v16)
    assert P.num_values == pv.size
    got_h = P.header[: G.num_tiles * 12].cpu().numpy().view(np.uint32).reshape(-1, 4, 3)
    assert np.array_equal(got_h, hdr)
    got_v = P.values[: P.num_values].view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got_v, pv)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N", [8, 32, 48, 128, 256, 300, 608])
@pytest.mark.parametrize("slabs", [None, 3])
def test_packed_spmm_bit_identical(cuda_device, dt, N, slabs):
    print(f"case packed dt={dt} N={N} slabs={slabs}", flush=True)
    G = _special_graph(cuda_device, dt, seed=N)
    P = core.pack_tiles(G.window_offset, G.original_col_indices, G.values_condensed, 16)
    plan = None if slabs is None else core.build_spmm_plan(G.window_offset, G.num_tiles, 16, slabs)
    X = synth.features(G.num_cols, N, seed=N + 2, device=cuda_device).to(dt)
    X[5] = float("inf")
    args = (G.window_offset, G.original_col_indices, G.values_condensed, X, 16)
    Yd = core.spmm(*args, plan=plan)
    Yp = core.spmm(*args, plan=plan, packed=P)
    torch.cuda.synchronize()
    assert torch.equal(_bits(Yd), _bits(Yp))


@pytest.mark.parametrize("waves", ["1", "2"])
def test_packed_spmm_waves_and_c2(cuda_device, waves):
    """c2 at full size, forced one- and two-wave work-groups, f16 values;
    the packed result also passes the oracle tolerance."""
    print(f"case packed c2 waves={waves}", flush=True)
    g = synth.config_graph("c2")
    win, cols, vals = core.csr_to_bcsr_cpu(g.num_nodes, g.row_ptr, g.col_idx, g.values, 16, 16)
    G = BCSRGraph(g.num_nodes, g.nnz, 16, 16, win, cols, vals, device=cuda_device, num_cols=g.num_nodes,
                  values_dtype=torch.float16)
    P = core.pack_tiles(G.window_offset, G.original_col_indices, G.values_condensed, 16)
    X = synth.features(g.num_nodes, 128, seed=3, device=cuda_device).to(torch.float16)
    args = (G.window_offset, G.original_col_indices, G.values_condensed, X, 16)
    from graph_rws_amd.core.ops import spmm_tuning
    with spmm_tuning(GRWS_SPMM_WAVES=int(waves)):
        Yd = core.spmm(*args)
        Yp = core.spmm(*args, packed=P)
        torch.cuda.synchronize()
    assert torch.equal(_bits(Yd), _bits(Yp))
    if waves == "1":
        Yr, Ya = oracle.bcsr_spmm(G.window_offset.cpu().numpy(), G.original_col_indices.cpu().numpy(),
                                  G.values_condensed.double().cpu().numpy(), 16, 16, X.double().cpu().numpy())
        err = np.abs(Yp.double().cpu().numpy() - Yr)
        assert (err <= 1e-2 * Ya).all()


def test_graph_packs_on_second_product_and_repacks_after_change(cuda_device):
    print("case pack policy", flush=True)
    G = _special_graph(cuda_device, torch.float16, seed=5)
    X = synth.features(G.num_cols, 64, seed=9, device=cuda_device).to(torch.float16)
    plan = G.spmm_plan(64)                        # the schedule G.spmm uses (split windows add in order)
    ref = core.spmm(G.window_offset, G.original_col_indices, G.values_condensed, X, 16, plan=plan)
    y1 = G.spmm(X)
    assert G._cache["packed"][2] is None          # first product: dense tiles
    y2 = G.spmm(X)
    P = G._cache["packed"][2]
    assert isinstance(P, core.PackedTiles)
    y3 = G.spmm(X)
    assert G._cache["packed"][2] is P              # reused
    for y in (y1, y2, y3):
        assert torch.equal(_bits(y), _bits(ref))
    with torch.no_grad():
        G.values_condensed.mul_(2)                 # in-place change: the packed copy is stale
    ref2 = core.spmm(G.window_offset, G.original_col_indices, G.values_condensed, X, 16, plan=plan)
    y4 = G.spmm(X)
    assert G._cache["packed"][2] is None
    y5 = G.spmm(X)
    assert G._cache["packed"][2] is not P
    torch.cuda.synchronize()
    assert torch.equal(_bits(y4), _bits(ref2)) and torch.equal(_bits(y5), _bits(ref2))


def test_packed_misaligned_x_and_refusals(cuda_device):
    """X rows that are not 16-byte aligned run the element-masked kernel on
    the dense values (same result); packing refuses 16x8 tiles and fp32
    values; grws_spmm_packed refuses values of another dtype than X."""
    print("case packed misaligned/refusals", flush=True)
    G = _special_graph(cuda_device, torch.bfloat16, seed=7)
    P = core.pack_tiles(G.window_offset, G.original_col_indices, G.values_condensed, 16)
    buf = synth.features(G.num_cols, 72, seed=4, device=cuda_device).to(torch.bfloat16)
    X = buf[:, 3:67]
    args = (G.window_offset, G.original_col_indices, G.values_condensed, X, 16)
    out_d = torch.empty(16 * G.num_windows, 64, dtype=torch.bfloat16, device=cuda_device)
    out_p = torch.empty_like(out_d)
    core.spmm(*args, out=out_d)
    core.spmm(*args, out=out_p, packed=P)
    torch.cuda.synchronize()
    assert torch.equal(_bits(out_d), _bits(out_p))
    assert core.pack_tiles(G.window_offset, G.original_col_indices.view(-1, 16)[:, :8].reshape(-1).contiguous(),
                           G.values_condensed[: G.num_tiles * 128].contiguous(), 8) is None
    assert core.pack_tiles(G.window_offset, G.original_col_indices, G.values_condensed.float(), 16) is None
    # values f32 with packed tiles: refused by the library
    vf = G.values_condensed.float()
    view = L.BcsrView(L.ptr(G.window_offset), L.ptr(G.original_col_indices), L.ptr(vf),
                      G.num_windows, G.num_tiles, 16, 16, L.GRWS_F32, 0)
    pk = P.view()
    Xc = X.contiguous()
    st = L.load().grws_spmm_packed(ctypes.byref(view), ctypes.byref(pk), None, L.ptr(Xc), L.GRWS_BF16,
                                   Xc.shape[0], Xc.stride(0), 64, L.ptr(out_p), L.GRWS_BF16, 64, None, 0,
                                   L.stream_of(cuda_device))
    assert st == L.GRWS_E_INVALID
