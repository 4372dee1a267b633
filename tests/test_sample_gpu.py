"""Node-wise sampler on the GPU (csrc/sample.hip) against the CPU oracle:
Philox draws, Floyd selection, relabel and the per-hop BCSR, bit for bit."""
import numpy as np
import pytest
import torch

import oracle
from graph_rws_amd import synth
from graph_rws_amd.core import relabel, sample_hop
from graph_rws_amd.core._lib import GrwsError
from graph_rws_amd.sampler import NeighborSampler

pytestmark = pytest.mark.gpu


def _csr(degs, n_ids, seed, device):
    rng = np.random.default_rng(seed)
    indptr = np.concatenate([[0], np.cumsum(degs)]).astype(np.int64)
    indices = rng.integers(0, n_ids, int(indptr[-1])).astype(np.int32)
    return (indptr, indices, torch.from_numpy(indptr).to(device),
            torch.from_numpy(indices).to(device))


DEGS = [0, 1, 2, 5, 6, 10, 15, 16, 31, 63, 64, 65, 100, 1000, 70000]


@pytest.mark.parametrize("k", [1, 5, 10, 15, 32, 64])
def test_sample_hop_bit_exact(cuda_device, k):
    degs = DEGS * 3
    ip, ix, ipd, ixd = _csr(degs, len(degs), 1, cuda_device)
    frontier = np.random.default_rng(k).permutation(len(degs)).astype(np.int64)
    dst, src, val = sample_hop(ipd, ixd, torch.from_numpy(frontier).to(cuda_device), k, seed=42)
    odst, osrc = oracle.sample_hop(ip, ix, 42, frontier, k)
    np.testing.assert_array_equal(dst.cpu().numpy(), odst)
    np.testing.assert_array_equal(src.cpu().numpy(), osrc)
    deg = ip[1:] - ip[:-1]
    oval = oracle.gcn_weight(deg[frontier[odst]], deg[osrc])
    np.testing.assert_array_equal(val.cpu().numpy(), oval)


def test_sample_hop_seeds_and_large_ids(cuda_device):
    # node ids above 2^32 are not possible with int32 indices, but the counter
    # uses both words of the id: check a graph large enough to span many
    # Philox counters and two different keys
    degs = np.random.default_rng(3).integers(0, 200, 20000)
    ip, ix, ipd, ixd = _csr(degs, 20000, 2, cuda_device)
    fr = np.random.default_rng(4).choice(20000, 5000, replace=False).astype(np.int64)
    for seed in (0, 42, 2 ** 63 + 12345):
        dst, src, _ = sample_hop(ipd, ixd, torch.from_numpy(fr).to(cuda_device), 15, seed=seed)
        odst, osrc = oracle.sample_hop(ip, ix, seed, fr, 15)
        np.testing.assert_array_equal(dst.cpu().numpy(), odst)
        np.testing.assert_array_equal(src.cpu().numpy(), osrc)


def test_sample_hop_empty_and_zero_degree(cuda_device):
    ip, ix, ipd, ixd = _csr([0, 0, 0], 3, 0, cuda_device)
    dst, src, val = sample_hop(ipd, ixd, torch.tensor([2, 0], device=cuda_device), 5)
    assert dst.numel() == 0 and src.numel() == 0
    dst, src, val = sample_hop(ipd, ixd, torch.empty(0, dtype=torch.int64, device=cuda_device), 5)
    assert dst.numel() == 0


def test_sample_hop_rejects_bad_input(cuda_device):
    ip, ix, ipd, ixd = _csr([3, 4], 2, 0, cuda_device)
    with pytest.raises(GrwsError, match="outside"):
        sample_hop(ipd, ixd, torch.tensor([0, 7], device=cuda_device), 2)
    with pytest.raises(GrwsError, match="fanout"):
        sample_hop(ipd, ixd, torch.tensor([0], device=cuda_device), 65)
    bad_ix = torch.tensor([0, 1, 9, 0, 1, 1, 0], dtype=torch.int32, device=cuda_device)
    with pytest.raises(GrwsError, match="neighbour index"):
        sample_hop(ipd, bad_ix, torch.tensor([0, 1], device=cuda_device), 5)
    bad_ip = torch.tensor([0, 5, 3], dtype=torch.int64, device=cuda_device)
    with pytest.raises(GrwsError, match="indptr"):
        sample_hop(bad_ip, ixd, torch.tensor([1], device=cuda_device), 2)


@pytest.mark.parametrize("F,E,n", [(1, 0, 10), (300, 4000, 5000), (5000, 100000, 10 ** 6),
                                   (0, 50, 100), (64, 64, 2 ** 27)])
def test_relabel_bit_exact(cuda_device, F, E, n):
    rng = np.random.default_rng(F + E)
    fr = rng.choice(n, F, replace=False).astype(np.int64) if F else np.empty(0, np.int64)
    src = rng.integers(0, n, E).astype(np.int64)
    if F and E:
        src[: E // 4] = fr[rng.integers(0, F, E // 4)]
    local, nxt = relabel(torch.from_numpy(fr).to(cuda_device), torch.from_numpy(src).to(cuda_device), n)
    olocal, onxt = oracle.relabel(fr, src)
    np.testing.assert_array_equal(nxt.cpu().numpy(), onxt)
    np.testing.assert_array_equal(local.cpu().numpy(), olocal)


def test_relabel_rejects_duplicate_frontier(cuda_device):
    fr = torch.tensor([4, 9, 4], device=cuda_device)
    with pytest.raises(GrwsError, match="twice"):
        relabel(fr, torch.tensor([1, 2], device=cuda_device), 10)
    with pytest.raises(GrwsError, match="outside"):
        relabel(torch.tensor([1], device=cuda_device), torch.tensor([10], device=cuda_device), 10)


def _check_blocks(blocks, ref, vdt):
    assert len(blocks) == len(ref)
    for b, r in zip(blocks, ref):
        assert b.num_rows == r["num_rows"] and b.num_cols == r["num_cols"]
        np.testing.assert_array_equal(b.src_nodes.cpu().numpy(), r["src_nodes"])
        np.testing.assert_array_equal(b.window_offset.cpu().numpy(), r["win"])
        np.testing.assert_array_equal(b.original_col_indices.cpu().numpy(), r["cols"])
        want = torch.from_numpy(r["vals"]).to(vdt)
        assert torch.equal(b.values_condensed.cpu(), want)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("tc,vdt", [(16, torch.float32), (8, torch.float32), (16, torch.float16),
                                    (16, torch.bfloat16)])
def test_neighbor_sampler_blocks_bit_exact(cuda_device, tc, vdt, fused):
    g = synth.c5_graph(device=cuda_device, scale=2e-4)  # 22k nodes, 320k edges
    seeds = synth.distinct_seeds(g.num_nodes, 256, seed=7, device=cuda_device)
    s = NeighborSampler([15, 10, 5], seed=42, tile_cols=tc, values_dtype=vdt, fused=fused)
    blocks = s.sample_layers(g.row_ptr, g.col_idx, seeds)
    ref = oracle.sample_blocks(g.row_ptr.cpu().numpy(), g.col_idx.cpu().numpy(),
                               seeds.cpu().numpy(), [15, 10, 5], seed=42, tile_cols=tc)
    _check_blocks(blocks, ref, vdt)


def test_fused_block_state_restored_and_fanout_64(cuda_device):
    """The dense relabel state is all -1 / all 0 after every call, also
    after a call that fails (duplicate frontier ids); fanout 64 (windows of
    up to 1,024 edges) matches the oracle."""
    from graph_rws_amd.core.ops import SampleState, sample_block
    degs = np.random.default_rng(6).integers(0, 300, 5000)
    ip, ix, ipd, ixd = _csr(degs, 5000, 7, cuda_device)
    st = SampleState(5000, cuda_device)
    fr = np.random.default_rng(8).choice(5000, 700, replace=False).astype(np.int64)
    win, cols, vals, nxt, E = sample_block(ipd, ixd, torch.from_numpy(fr).to(cuda_device), 64, st)
    ref = oracle.sample_blocks(ip, ix, fr, [64], seed=42, tile_cols=16)[0]
    np.testing.assert_array_equal(nxt.cpu().numpy(), ref["src_nodes"])
    np.testing.assert_array_equal(win.cpu().numpy(), ref["win"])
    np.testing.assert_array_equal(cols.cpu().numpy(), ref["cols"])
    np.testing.assert_array_equal(vals.cpu().numpy(), ref["vals"])
    assert E == ref["dst"].size
    assert bool((st.node_map == -1).all()) and bool((st.bitmap == 0).all())
    bad = torch.tensor([3, 9, 3], device=cuda_device)
    with pytest.raises(GrwsError, match="twice"):
        sample_block(ipd, ixd, bad, 5, st)
    assert bool((st.node_map == -1).all()) and bool((st.bitmap == 0).all())


def test_neighbor_sampler_c5_batch_shape(cuda_device):
    """A full-size c5 batch (1,024 seeds, fanouts [15,10,5]) on a graph with
    c5's degree law at 1/20 of its node count: bit-exact against the oracle,
    plus the size-independent invariants."""
    g = synth.c5_graph(device=cuda_device, scale=0.05)
    seeds = synth.distinct_seeds(g.num_nodes, 1024, seed=42, device=cuda_device)
    s = NeighborSampler([15, 10, 5], seed=42, tile_cols=16)
    blocks = s.sample_layers(g.row_ptr, g.col_idx, seeds)
    ip = g.row_ptr.cpu().numpy()
    ref = oracle.sample_blocks(ip, g.col_idx.cpu().numpy(), seeds.cpu().numpy(), [15, 10, 5])
    _check_blocks(blocks, ref, torch.float32)
    deg = ip[1:] - ip[:-1]
    for b in blocks:  # every destination got min(deg, k) edges
        dnodes = b.dst_nodes.cpu().numpy()
        got = np.diff(b.window_offset.cpu().numpy())  # tiles only; count edges via COO instead
        assert got.sum() == b.num_tiles
        want = np.minimum(deg[dnodes], b.fanout).sum()
        assert b.num_sampled_edges == want


@pytest.mark.parametrize("hops,tc", [([5, 10, 15], 16), ([5, 10, 15], 8), ([64, 1], 16), ([2] * 8, 16),
                                     ([1], 16)])
def test_sample_blocks_one_call_bit_exact(cuda_device, hops, tc):
    """grws_sample_blocks (every hop of the batch in one call, fanouts in hop
    order): each hop equal, bit for bit, to the oracle's; the dense state is
    all -1 / all 0 afterwards; zero-degree and hub nodes included."""
    from graph_rws_amd.core.ops import SampleState, sample_blocks
    degs = np.random.default_rng(16).integers(0, 40, 6000)
    degs[::97] = 0
    degs[5] = 3000
    ip, ix, ipd, ixd = _csr(degs, 6000, 17, cuda_device)
    st = SampleState(6000, cuda_device)
    seeds = np.random.default_rng(18).choice(6000, 300, replace=False).astype(np.int64)
    seeds[0] = 5
    out = sample_blocks(ipd, ixd, torch.from_numpy(seeds).to(cuda_device), hops, st, seed=42, tile_cols=tc)
    ref = oracle.sample_blocks(ip, ix, seeds, list(reversed(hops)), seed=42, tile_cols=tc)[::-1]
    assert len(out) == len(ref) == len(hops)
    for h, ((win, cols, vals, nxt, E), r) in enumerate(zip(out, ref)):
        np.testing.assert_array_equal(nxt.cpu().numpy(), r["src_nodes"], err_msg=f"hop {h}")
        np.testing.assert_array_equal(win.cpu().numpy(), r["win"], err_msg=f"hop {h}")
        np.testing.assert_array_equal(cols.cpu().numpy(), r["cols"], err_msg=f"hop {h}")
        np.testing.assert_array_equal(vals.cpu().numpy(), r["vals"], err_msg=f"hop {h}")
        assert E == r["dst"].size
    assert bool((st.node_map == -1).all()) and bool((st.bitmap == 0).all())
    # the same state serves the next batch (and the per-hop entry point)
    out2 = sample_blocks(ipd, ixd, torch.from_numpy(seeds[::-1].copy()).to(cuda_device), hops, st, tile_cols=tc)
    ref2 = oracle.sample_blocks(ip, ix, seeds[::-1].copy(), list(reversed(hops)), tile_cols=tc)[::-1]
    for (win, cols, vals, nxt, E), r in zip(out2, ref2):
        np.testing.assert_array_equal(cols.cpu().numpy(), r["cols"])
        np.testing.assert_array_equal(nxt.cpu().numpy(), r["src_nodes"])


def test_sample_blocks_errors_leave_state_clean(cuda_device):
    """Duplicate or out-of-range seeds are reported after the batch (the
    kernels skip them); the state is restored, and the empty batch is a
    no-op."""
    from graph_rws_amd.core.ops import SampleState, sample_blocks
    ip, ix, ipd, ixd = _csr([3, 4, 0, 2, 5], 5, 0, cuda_device)
    st = SampleState(5, cuda_device)
    with pytest.raises(GrwsError, match="twice"):
        sample_blocks(ipd, ixd, torch.tensor([1, 3, 1], device=cuda_device), [2, 2], st)
    assert bool((st.node_map == -1).all()) and bool((st.bitmap == 0).all())
    with pytest.raises(GrwsError, match="outside"):
        sample_blocks(ipd, ixd, torch.tensor([0, 11], device=cuda_device), [3], st)
    assert bool((st.node_map == -1).all()) and bool((st.bitmap == 0).all())
    out = sample_blocks(ipd, ixd, torch.empty(0, dtype=torch.int64, device=cuda_device), [3, 3], st)
    for win, cols, vals, nxt, E in out:
        assert E == 0 and nxt.numel() == 0 and win.cpu().tolist() == [0]
    bad_ix = torch.tensor([0, 1, 9, 0, 1, 1, 0, 2, 2, 3, 3, 4, 4, 0], dtype=torch.int32, device=cuda_device)
    with pytest.raises(GrwsError, match="neighbour index"):
        sample_blocks(ipd, bad_ix, torch.tensor([0, 1], device=cuda_device), [5], st)
    assert bool((st.node_map == -1).all()) and bool((st.bitmap == 0).all())


def _vdt_cast(vals: np.ndarray, vdt) -> np.ndarray:
    if vdt == torch.float16:
        return vals.astype(np.float16)
    if vdt == torch.bfloat16:
        return oracle.round_to_bf16(vals.astype(np.float32))
    return vals.astype(np.float32)


def _tensor_np(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.float().cpu().numpy()
    return t.cpu().numpy()


@pytest.mark.parametrize("hops,tc,vdt,mask", [([5, 10, 15], 16, torch.float32, None),
                                              ([5, 10, 15], 8, torch.float16, None),
                                              ([5, 10, 15], 16, torch.bfloat16, [True, False, True]),
                                              ([64, 1], 16, torch.float32, None),
                                              ([2] * 8, 16, torch.float16, None)])
def test_sample_blocks_transposed_bit_exact(cuda_device, hops, tc, vdt, mask):
    """grws_sample_blocks_transposed: the blocks are those of the plain call,
    and each transposed block equals, bit for bit, the oracle's BCSR of the
    hop's edges with rows and columns swapped (sources as rows, the
    frontier rows as columns: the reference converter's layout), and the
    device build of the block's transpose (builder.transpose).  Hub and
    zero-degree nodes included; a repeated (row, source) pair keeps one
    entry."""
    from graph_rws_amd import builder
    from graph_rws_amd.core.ops import SampleState, sample_blocks
    from graph_rws_amd.data import BCSRGraph
    degs = np.random.default_rng(16).integers(0, 40, 6000)
    degs[::97] = 0
    degs[5] = 3000
    ip, ix, ipd, ixd = _csr(degs, 6000, 17, cuda_device)
    st = SampleState(6000, cuda_device)
    seeds = np.random.default_rng(18).choice(6000, 300, replace=False).astype(np.int64)
    seeds[0] = 5
    sd = torch.from_numpy(seeds).to(cuda_device)
    mask = mask or [True] * len(hops)
    out = sample_blocks(ipd, ixd, sd, hops, st, seed=42, tile_cols=tc, values_dtype=vdt, transposes=mask)
    plain = sample_blocks(ipd, ixd, sd, hops, st, seed=42, tile_cols=tc, values_dtype=vdt)
    ref = oracle.sample_blocks(ip, ix, seeds, list(reversed(hops)), seed=42, tile_cols=tc)[::-1]
    for h, (o, p, r) in enumerate(zip(out, plain, ref)):
        for a, b in zip(o[:4], p[:4]):
            np.testing.assert_array_equal(_tensor_np(a), _tensor_np(b), err_msg=f"hop {h}")
        assert o[4] == p[4]
        if not mask[h]:
            assert o[5] is None
            continue
        twin, tcols, tvals, tmax = o[5]
        S = r["num_cols"]
        ow, oc, ov = oracle.coo_to_bcsr(S, r["src_local"], r["dst"], r["val"], tc)
        np.testing.assert_array_equal(twin.cpu().numpy(), ow, err_msg=f"hop {h}: t_window_offset")
        np.testing.assert_array_equal(tcols.cpu().numpy(), oc, err_msg=f"hop {h}: t_col_indices")
        np.testing.assert_array_equal(_tensor_np(tvals), _vdt_cast(ov, vdt).astype(np.float32)
                                      if vdt == torch.bfloat16 else _vdt_cast(ov, vdt), err_msg=f"hop {h}: t_values")
        assert tmax == int(np.diff(ow).max(initial=0))
        # the device build of the block's transpose gives the same arrays
        win, cols, vals = o[0], o[1], o[2]
        F = r["num_rows"]
        g = BCSRGraph(num_nodes=F, num_edges=o[4], tile_rows=16, tile_cols=tc, window_offset=win,
                      original_col_indices=cols, values_condensed=vals, device=cuda_device, num_rows=F,
                      num_cols=S, values_dtype=vdt)
        AT = builder.transpose(g)
        np.testing.assert_array_equal(AT.window_offset.cpu().numpy(), twin.cpu().numpy())
        np.testing.assert_array_equal(AT.original_col_indices.cpu().numpy(), tcols.cpu().numpy())
        np.testing.assert_array_equal(_tensor_np(AT.values_condensed), _tensor_np(tvals))
    assert bool((st.node_map == -1).all()) and bool((st.bitmap == 0).all())


def test_neighbor_sampler_blocks_carry_their_transposes(cuda_device):
    """sample_layers(transposes=...) attaches each built transpose to its
    block: transpose() returns it without a build, and the backward SpMM
    over it equals the one over a fresh device build."""
    g = synth.c5_graph(device=cuda_device, scale=1e-4)
    seeds = synth.distinct_seeds(g.num_nodes, 200, seed=3, device=cuda_device)
    s = NeighborSampler([6, 4, 3], tile_cols=16, values_dtype=torch.float16)
    blocks = s.sample_layers(g.row_ptr, g.col_idx, seeds, transposes=[False, True, True])
    assert blocks[0]._cache.get("T") is None
    from graph_rws_amd import builder
    for b in blocks[1:]:
        AT = b.transpose()
        assert AT is b._cache["T"][1]
        fresh = builder.transpose(b)
        np.testing.assert_array_equal(AT.window_offset.cpu().numpy(), fresh.window_offset.cpu().numpy())
        np.testing.assert_array_equal(AT.original_col_indices.cpu().numpy(),
                                      fresh.original_col_indices.cpu().numpy())
        np.testing.assert_array_equal(AT.values_condensed.cpu().numpy(), fresh.values_condensed.cpu().numpy())
        assert AT.max_window_slabs == fresh.max_window_slabs
        G = torch.randn(16 * b.num_windows, 32, device=cuda_device).half()
        torch.testing.assert_close(AT.spmm(G), fresh.spmm(G), rtol=0, atol=0)
