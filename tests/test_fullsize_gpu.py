"""The benchmarked workloads at their full BASELINE sizes against the float64
oracle (tests/_fullsize.py: a fixed window set elementwise, and a projection
over every row), through the same calls bench.py times.

* c3 (232,965 nodes, 114.6M nnz, f16): the headline N=608 product on X at a
  640-element pitch, default plan, chunk-major order, the dense-tile first
  product, the 4-window grouped second product and the packed-tile product
  (bit-identical to the dense one); the epoch widths N=256 (window by
  window, then 4-window groups) and N=41 (ragged); A^T G at N=256 (first
  product window by window, second on 4-window groups); the same graph in
  bf16 at N=256 (the bf16 slab-pair kernel).  Every grouped product is also
  compared with the window-by-window one over the whole output.
* c4 (2,449,029 nodes, 123.7M nnz, bf16): N=112 at a 128-element pitch,
  N=256 (two 128-column chunks), N=47 (ragged); A^T G at N=256.
* c2 (169,343 nodes, 2.33M nnz): A^T G at N=128 in f16 and bf16 through the
  cached transpose, as the bench's backward leg.
* c5 (111M nodes, 1.6B edges): one full-size sampling batch bit-exact
  against the host sampler driven by the same Philox draws.

Tolerance (north_star): rtol 1e-2 for f16/bf16 inputs against |A| |X|,
and the tight tier of tests/_fullsize.py (the arithmetic's own bound).
The forward semantics follow /root/reference/core/include/spmm_tc.cuh:113-193
(every output column computed, -1 slots skipped), the transpose :238-269
without its atomics and 1e-9 skip, the sampling hop order
/root/reference/sampler/sampler.py:186-279.
"""
import numpy as np
import pytest
import torch

import oracle
from _fullsize import HostGraph, check_forward, check_transpose
from graph_rws_amd import synth
from graph_rws_amd.data import BCSRGraph, aligned_rows

pytestmark = pytest.mark.gpu

RTOL = 1e-2


def _graph(cfg, dev, vdt):
    g = synth.config_graph(cfg, device=dev)
    G = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes, tile_cols=16,
                           device=dev, values_dtype=vdt)
    torch.cuda.synchronize()
    return g, G


@pytest.fixture(scope="module")
def c3(cuda_device):
    print("fixture c3 full size (f16)", flush=True)
    g, G = _graph("c3", cuda_device, torch.float16)
    return g, G, HostGraph(G)


@pytest.fixture(scope="module")
def c4(cuda_device):
    print("fixture c4 full size (bf16)", flush=True)
    g, G = _graph("c4", cuda_device, torch.bfloat16)
    return g, G, HostGraph(G)


def test_c3_headline_n608_bench_path(c3, cuda_device, monkeypatch):
    """bench.py's timed call: X [n, 608] f16 at a 640 pitch, Y preallocated,
    G.spmm(X, out=Y).  The first product runs window by window on the dense
    tiles; the second builds and reads the grouped tiles (c3 has community
    structure: 4 windows need 54% of their own column slots), the product
    bench.py times; with grouping off the packed tiles give the first
    product's bits."""
    from graph_rws_amd.core import ops
    print("case c3 N=608 f16 bench path", flush=True)
    g, G, hg = c3
    X = aligned_rows(synth.features(g.num_nodes, 602, pad_to=608, seed=7, device=cuda_device).half())
    assert X.stride(0) == 640
    plan = G.spmm_plan(608)
    Y1 = torch.empty((16 * G.num_windows, 608), dtype=torch.float16, device=cuda_device)
    Y2 = torch.empty_like(Y1)
    G.spmm(X, out=Y1)
    G.spmm(X, out=Y2)
    torch.cuda.synchronize()
    gt = G.grouped_tiles(X.shape[0], 608)
    assert gt is not None and gt.slot_ratio < ops.GROUP_MAX_RATIO, "c3 must take the grouped tiles"
    assert gt.group_size == 4
    print("grouped tiles: 4 windows, slot ratio", round(gt.slot_ratio, 4), flush=True)
    print(check_forward(hg, X, Y2, RTOL, plan=plan, seed=3), flush=True)
    print(check_forward(hg, X, Y1, RTOL, plan=plan, seed=4), flush=True)
    monkeypatch.setattr(ops, "GROUPED", False)
    Y3 = torch.empty_like(Y1)
    G.spmm(X, out=Y3)
    torch.cuda.synchronize()
    assert G.packed_tiles() is not None, "the packed tiles are built on the next product"
    assert torch.equal(Y1.view(torch.int16), Y3.view(torch.int16)), "packed and dense tiles differ"
    Ya = G.spmm(X.abs())
    torch.cuda.synchronize()
    print("grouped vs window by window, worst of bound:", _compare_orders(G, hg, X, Ya, Y2, Y1), flush=True)


def _record_grouped(monkeypatch):
    """Records, for every SpMM entry point the shim calls, its name and the
    group size of the grouped tiles it was handed (None otherwise)."""
    from graph_rws_amd.core import ops
    calls = []
    real = ops.L.call

    def spy(fn, *args):
        gs = None
        if fn == "grws_spmm_grouped":
            gs = args[1]._obj.group_size
        if fn.startswith("grws_spmm"):
            calls.append((fn, gs))
        return real(fn, *args)

    monkeypatch.setattr(ops.L, "call", spy)
    return calls


def _compare_orders(G, hg, X, Ya_x, Yg, Yw):
    """The grouped product Yg against the window-by-window product Yw over
    every output element: both round the same exact sum once to the output
    type (f16 or bf16) after fp32 accumulations in different orders, so they
    differ by at most u_out (|Yg| + |Yw|) + 2 C k 2^-24 (|A||X|) (+ subnormal
    and flush terms), with |A||X| from the device product of A and |X|
    (A >= 0 on these graphs; Ya_x is rounded to the output type, hence the
    factor 1 + 4 u_out on it)."""
    from _fullsize import C_SUM_16, DT, FTZ, S_OUT, U32, U_OUT, all_row_nnz
    dt = DT[Yg.dtype]
    k = torch.from_numpy(all_row_nnz(hg)).to(Yg.device, torch.float32)[:, None]
    ya = Ya_x.float() * (1 + 4 * U_OUT[dt])
    d = (Yg.float() - Yw.float()).abs()
    bound = (U_OUT[dt] * (Yg.float().abs() + Yw.float().abs()) + 2 * C_SUM_16 * U32 * k * ya
             + 2 * (k * FTZ + S_OUT[dt]))
    bad = d > bound
    assert not bool(bad.any()), f"grouped vs window by window: {int(bad.sum())} of {bad.numel()} apart"
    return float((d / bound).max())


def test_c3_epoch_n256_grouped_4_windows(c3, cuda_device, monkeypatch):
    """The c3 epoch's 256-column products: the first runs window by window,
    the second builds and reads 4-window grouped tiles (the layout the
    epoch's hidden layers use, spmm_grp_kernel with 4 waves), both checked
    against the oracle in both tiers, and the two compared over the whole
    output (semantics: /root/reference/core/include/spmm_tc.cuh:113-193)."""
    from graph_rws_amd.core import ops
    print("case c3 N=256 f16 window by window, then 4-window groups", flush=True)
    g, G, hg = c3
    X = synth.features(g.num_nodes, 256, seed=256, device=cuda_device).half()
    calls = _record_grouped(monkeypatch)
    Y1 = G.spmm(X)
    Y2 = G.spmm(X)
    torch.cuda.synchronize()
    gt = G.grouped_tiles(X.shape[0], 256)
    assert gt is not None and gt.group_size == 4, "c3 at N=256 must take 4-window grouped tiles"
    assert ("grws_spmm_grouped", 4) in calls, calls
    print(check_forward(hg, X, Y2, RTOL, plan=G.spmm_plan(256), seed=256), flush=True)
    Yw = Y1 if calls[0][0] != "grws_spmm_grouped" else None
    if Yw is None:  # an earlier product made this the grouped one: force window by window
        monkeypatch.setattr(ops, "GROUPED", False)
        Yw = G.spmm(X)
        monkeypatch.setattr(ops, "GROUPED", True)
    print(check_forward(hg, X, Yw, RTOL, plan=G.spmm_plan(256), seed=257), flush=True)
    monkeypatch.setattr(ops, "GROUPED", False)
    Ya = G.spmm(X.abs())
    torch.cuda.synchronize()
    print("grouped vs window by window, worst of bound:", _compare_orders(G, hg, X, Ya, Y2, Yw), flush=True)


def test_c3_epoch_n41(c3, cuda_device):
    print("case c3 N=41 f16", flush=True)
    g, G, hg = c3
    X = synth.features(g.num_nodes, 41, seed=41, device=cuda_device).half()
    Y = G.spmm(X)
    torch.cuda.synchronize()
    assert Y.shape == (16 * G.num_windows, 41)
    print(check_forward(hg, X, Y, RTOL, plan=G.spmm_plan(41), seed=41), flush=True)


def test_c3_transpose_n256(c3, cuda_device, monkeypatch):
    """A^T G through the cached transpose, as the epoch's backward makes it:
    the first product window by window, the second (and every later one)
    on the transpose's own 4-window grouped tiles; both against the oracle
    on A (/root/reference/core/include/spmm_tc.cuh:238-269 semantics,
    without its atomics and 1e-9 skip)."""
    print("case c3 A^T G N=256 f16, first and second product", flush=True)
    g, G, hg = c3
    Gout = synth.features(16 * G.num_windows, 256, seed=31, device=cuda_device).half()
    calls = _record_grouped(monkeypatch)
    out1 = G.spmm_transpose(Gout)
    out2 = G.spmm_transpose(Gout)
    torch.cuda.synchronize()
    AT = G.transpose()
    assert ("grws_spmm_grouped", 4) in calls, calls
    assert AT.grouped_tiles(Gout.shape[0], 256).group_size == 4
    hgT = HostGraph(AT)
    print(check_transpose(hg, hgT, Gout, out2, RTOL, planT=AT.spmm_plan(256), seed=5), flush=True)
    print(check_transpose(hg, hgT, Gout, out1, RTOL, planT=AT.spmm_plan(256), seed=6), flush=True)


def test_c3_bf16_n256_slab_pairs(c3, cuda_device, monkeypatch):
    """The c3 graph with bf16 values and X (the 16-bit type c4 is configured
    in) at N=256: the second product runs the 4-window grouped tiles on the
    bf16 slab-pair kernel (v_mfma_f32_16x16x32_bf16); against the oracle in
    both tiers and against the window-by-window product over the whole
    output (semantics: /root/reference/core/include/spmm_tc.cuh:113-193)."""
    from graph_rws_amd.core import ops
    print("case c3 N=256 bf16, 4-window groups on slab pairs", flush=True)
    g, G16, _ = c3
    G = G16.with_values_dtype(torch.bfloat16)
    hg = HostGraph(G)
    X = synth.features(g.num_nodes, 256, seed=612, device=cuda_device).to(torch.bfloat16)
    calls = _record_grouped(monkeypatch)
    G.spmm(X)
    Y2 = G.spmm(X)
    torch.cuda.synchronize()
    assert ("grws_spmm_grouped", 4) in calls, calls
    assert ops.grouped_slab_pairs(), "4-window groups run slab pairs by default"
    print(check_forward(hg, X, Y2, RTOL, plan=G.spmm_plan(256), seed=612), flush=True)
    monkeypatch.setattr(ops, "GROUPED", False)
    Yw = G.spmm(X)
    Ya = G.spmm(X.abs())
    torch.cuda.synchronize()
    print("grouped vs window by window, worst of bound:", _compare_orders(G, hg, X, Ya, Y2, Yw), flush=True)


@pytest.mark.parametrize("N,d", [(608, 602), (256, 256)])
def test_c3_grouped_product_repeats_bit_identically(c3, cuda_device, N, d):
    """The grouped product's direct loads into LDS against a race: at full
    size (3,641 groups, 320-column chunks at N=608, 3 work-groups per CU),
    twenty products in a row equal the first bit for bit, and equal the
    register-staged kernel's (GRWS_GRP_DMA=0): the same sums in the same
    order.  A pair's rows read before every wave's loads had landed gave
    results that changed from run to run."""
    from graph_rws_amd.core import ops
    print(f"case c3 N={N} grouped product repeated", flush=True)
    g, G, _ = c3
    X = aligned_rows(synth.features(g.num_nodes, d, pad_to=N, seed=N + 3, device=cuda_device).half())
    gt = G.grouped_tiles(X.shape[0], N)
    if gt is None:  # built on the graph's second product of this width
        G.spmm(X)
        gt = G.grouped_tiles(X.shape[0], N)
    assert gt is not None and gt.group_size == 4
    assert ops.grouped_kernel(4) == "spmm_grp2d_kernel"
    Y0 = ops.spmm(G.window_offset, G.original_col_indices, G.values_condensed, X, 16, grouped=gt)
    same = 0
    for _ in range(20):
        Y = ops.spmm(G.window_offset, G.original_col_indices, G.values_condensed, X, 16, grouped=gt)
        same += bool(torch.equal(Y.view(torch.int16), Y0.view(torch.int16)))
    with ops.spmm_tuning(GRWS_GRP_DMA=0):
        Yr = ops.spmm(G.window_offset, G.original_col_indices, G.values_condensed, X, 16, grouped=gt)
    torch.cuda.synchronize()
    assert same == 20, f"{20 - same} of 20 repeats differ"
    assert torch.equal(Yr.view(torch.int16), Y0.view(torch.int16))


def test_c4_bench_path_n112(c4, cuda_device):
    """X [n, 112] bf16 at a 128-element (256-byte) pitch, as bench.py
    --config c4 and the aggregate-first layer 0 gather it."""
    print("case c4 N=112 bf16", flush=True)
    g, G, hg = c4
    X = aligned_rows(synth.features(g.num_nodes, 100, pad_to=112, seed=7, device=cuda_device).to(torch.bfloat16))
    assert X.stride(0) == 128
    Y1 = G.spmm(X)
    Y2 = G.spmm(X)
    torch.cuda.synchronize()
    assert torch.equal(Y1.view(torch.int16), Y2.view(torch.int16))
    print(check_forward(hg, X, Y2, RTOL, plan=G.spmm_plan(112), seed=7), flush=True)


@pytest.mark.parametrize("N", [256, 47])
def test_c4_epoch_widths(c4, cuda_device, N):
    print(f"case c4 N={N} bf16", flush=True)
    g, G, hg = c4
    X = synth.features(g.num_nodes, N, seed=N, device=cuda_device).to(torch.bfloat16)
    Y = G.spmm(X)
    torch.cuda.synchronize()
    print(check_forward(hg, X, Y, RTOL, plan=G.spmm_plan(N), seed=N), flush=True)


def test_c4_transpose_n256(c4, cuda_device):
    print("case c4 A^T G N=256 bf16", flush=True)
    g, G, hg = c4
    Gout = synth.features(16 * G.num_windows, 256, seed=41, device=cuda_device).to(torch.bfloat16)
    out = G.spmm_transpose(Gout)
    torch.cuda.synchronize()
    AT = G.transpose()
    print(check_transpose(hg, HostGraph(AT), Gout, out, RTOL, planT=AT.spmm_plan(256), seed=9), flush=True)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_c2_transpose_bench_leg(cuda_device, dt):
    """bench.py's c2 backward leg: AT = G.transpose(); AT.spmm(G_r, out=)."""
    print(f"case c2 A^T G N=128 {dt}", flush=True)
    g, G = _graph("c2", cuda_device, dt)
    Gr = synth.features(16 * G.num_windows, 128, seed=22, device=cuda_device).to(dt)
    AT = G.transpose()
    out = torch.empty((16 * AT.num_windows, 128), dtype=dt, device=cuda_device)
    for _ in range(3):  # plan, then packed tiles, then the packed product
        AT.spmm(Gr, out=out)
    torch.cuda.synchronize()
    print(check_transpose(HostGraph(G), HostGraph(AT), Gr, out[: g.num_nodes], RTOL,
                          planT=AT.spmm_plan(128), seed=2), flush=True)


def test_c5_full_size_batch_bit_exact(cuda_device):
    """One c5 batch (1,024 seeds, fanouts [15, 10, 5], Philox seed 42) on the
    111M-node graph: every per-hop block equal, bit for bit, to the host
    sampler's."""
    print("case c5 full-size batch", flush=True)
    from graph_rws_amd.sampler import NeighborSampler
    c = synth.C5
    g = synth.c5_graph(device=cuda_device)
    s = NeighborSampler(c["fanouts"], seed=c["philox_seed"], tile_cols=16)
    seeds = synth.distinct_seeds(g.num_nodes, c["batch"], seed=1000, device=cuda_device)
    blocks = s.sample_layers(g.row_ptr, g.col_idx, seeds)
    torch.cuda.synchronize()
    ref = oracle.sample_blocks(g.row_ptr.cpu().numpy(), g.col_idx.cpu().numpy(), seeds.cpu().numpy(),
                               c["fanouts"], seed=c["philox_seed"], tile_cols=16)
    assert len(blocks) == len(ref) == 3
    for i, (b, r) in enumerate(zip(blocks, ref)):
        np.testing.assert_array_equal(b.src_nodes.cpu().numpy(), r["src_nodes"], err_msg=f"hop {i} src")
        np.testing.assert_array_equal(b.window_offset.cpu().numpy(), r["win"], err_msg=f"hop {i} win")
        np.testing.assert_array_equal(b.original_col_indices.cpu().numpy(), r["cols"], err_msg=f"hop {i} cols")
        np.testing.assert_array_equal(b.values_condensed.cpu().numpy(), r["vals"], err_msg=f"hop {i} vals")
    assert sum(int(r["dst"].size) for r in ref) > 300_000
