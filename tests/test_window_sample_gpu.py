"""Window top-K sampler on the GPU (csrc/window_sample.hip) against the CPU
restatement of the reference's sampling kernels, bit for bit."""
import numpy as np
import pytest
import torch

import oracle
from graph_rws_amd import synth
from graph_rws_amd.core import sample_all_layers, window_seeds
from graph_rws_amd.core._lib import GrwsError
from graph_rws_amd.data import BCSRGraph
from graph_rws_amd.sampler import BCSRSampler

pytestmark = pytest.mark.gpu


def _graph(name, dev, tc=8, scale=1.0, vdt=torch.float32):
    g = synth.config_graph(name, scale=scale)
    G = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes,
                           tile_cols=tc, device=dev, values_dtype=vdt)
    return g, G


def _compare(layers, ref, vdt=torch.float32):
    assert len(layers) == len(ref)
    for got, want in zip(layers, ref):
        ow, oc, ov, act, msk = got
        rw, rc, rv, ract, rmsk = want
        np.testing.assert_array_equal(act.cpu().numpy(), ract)
        np.testing.assert_array_equal(msk.cpu().numpy(), rmsk)
        np.testing.assert_array_equal(ow.cpu().numpy(), rw)
        np.testing.assert_array_equal(oc.cpu().numpy(), rc)
        assert torch.equal(ov.cpu(), torch.from_numpy(rv).to(vdt))


@pytest.mark.parametrize("fanouts", [[5], [10, 10], [15, 10, 5], [32, 40], [100, 129], [256]])
def test_sample_all_layers_c1_bit_exact(cuda_device, fanouts):
    g, G = _graph("c1", cuda_device)
    seeds = np.random.default_rng(len(fanouts)).choice(g.num_nodes, 300, replace=False)
    layers, timings = sample_all_layers(G.window_offset, G.original_col_indices,
                                        G.values_condensed, torch.from_numpy(seeds).to(cuda_device),
                                        fanouts, g.num_nodes, None, None, None, None)
    ref = oracle.window_sample_all_layers(G.window_offset.cpu().numpy(),
                                          G.original_col_indices.cpu().numpy(),
                                          G.values_condensed.cpu().numpy(), seeds, fanouts,
                                          g.num_nodes)
    _compare(layers, ref)
    assert len(timings) == len(fanouts) and all(t.total_time >= 0 for t in timings)


def test_sample_all_layers_c2_full_size(cuda_device):
    """1,024 seeds over the full c2 graph (169k nodes), fanouts [15,10,5] in
    the reference's sampling order (5 first)."""
    g, G = _graph("c2", cuda_device)
    seeds = synth.distinct_seeds(g.num_nodes, 1024, seed=3).numpy()
    layers, _ = sample_all_layers(G.window_offset, G.original_col_indices, G.values_condensed,
                                  torch.from_numpy(seeds).to(cuda_device), [5, 10, 15],
                                  g.num_nodes)
    ref = oracle.window_sample_all_layers(G.window_offset.cpu().numpy(),
                                          G.original_col_indices.cpu().numpy(),
                                          G.values_condensed.cpu().numpy(), seeds, [5, 10, 15],
                                          g.num_nodes)
    _compare(layers, ref)


def test_sample_all_layers_c3_dense_windows(cuda_device):
    """Dense community windows (thousands of candidate columns per window):
    the radix select resolves many equal totals by column."""
    g, G = _graph("c3", cuda_device, scale=0.02)
    seeds = synth.distinct_seeds(g.num_nodes, 256, seed=5).numpy()
    for fanouts in ([10, 25], [100], [200]):
        layers, _ = sample_all_layers(G.window_offset, G.original_col_indices,
                                      G.values_condensed, torch.from_numpy(seeds).to(cuda_device),
                                      fanouts, g.num_nodes)
        ref = oracle.window_sample_all_layers(G.window_offset.cpu().numpy(),
                                              G.original_col_indices.cpu().numpy(),
                                              G.values_condensed.cpu().numpy(), seeds, fanouts,
                                              g.num_nodes)
        _compare(layers, ref)


@pytest.mark.parametrize("vdt", [torch.float16, torch.bfloat16])
def test_sample_all_layers_low_precision_values(cuda_device, vdt):
    g, G = _graph("c1", cuda_device, vdt=vdt)
    seeds = np.arange(0, g.num_nodes, 5)
    layers, _ = sample_all_layers(G.window_offset, G.original_col_indices, G.values_condensed,
                                  torch.from_numpy(seeds).to(cuda_device), [20, 7], g.num_nodes)
    ref = oracle.window_sample_all_layers(G.window_offset.cpu().numpy(),
                                          G.original_col_indices.cpu().numpy(),
                                          G.values_condensed.float().cpu().numpy(), seeds,
                                          [20, 7], g.num_nodes)
    _compare(layers, ref, vdt)


def test_sample_all_layers_hacs_locality(cuda_device):
    g, G = _graph("c1", cuda_device)
    rng = np.random.default_rng(4)
    q = rng.random(g.num_nodes).astype(np.float32)
    q[rng.random(g.num_nodes) < 0.1] = 0.0
    W = G.num_windows
    parts = np.array([[0, 900], [900, 1800], [1800, 2708]], np.int32)
    wpart = rng.integers(-1, 3, W).astype(np.int32)
    seeds = np.arange(3, g.num_nodes, 9)
    kw = dict(alpha=0.5, beta=3.0, delta=0.25, gamma_bonus=0.37, score_scale=250.0)
    layers, _ = sample_all_layers(
        G.window_offset, G.original_col_indices, G.values_condensed,
        torch.from_numpy(seeds).to(cuda_device), [12, 40], g.num_nodes,
        torch.from_numpy(q).to(cuda_device), torch.from_numpy(wpart).to(cuda_device),
        torch.from_numpy(parts[:, 0].copy()).to(cuda_device),
        torch.from_numpy(parts[:, 1].copy()).to(cuda_device), use_hacs=1, locality_enabled=1, **kw)
    hacs = dict(static_scores=q, window_part_ids=wpart, part_starts=parts[:, 0],
                part_ends=parts[:, 1], use_hacs=1, locality_enabled=1, **kw)
    ref = oracle.window_sample_all_layers(G.window_offset.cpu().numpy(),
                                          G.original_col_indices.cpu().numpy(),
                                          G.values_condensed.cpu().numpy(), seeds, [12, 40],
                                          g.num_nodes, hacs=hacs)
    _compare(layers, ref)


def test_window_seeds_matches_oracle(cuda_device):
    rng = np.random.default_rng(9)
    ids = rng.integers(-1, 5000, 20000).astype(np.int32)
    act, msk = window_seeds(torch.from_numpy(ids).to(cuda_device), 5000)
    ra, rm = oracle.prepare_windows(ids)
    np.testing.assert_array_equal(act.cpu().numpy(), ra)
    np.testing.assert_array_equal(msk.cpu().numpy(), rm)


def test_sample_all_layers_rejects_bad_input(cuda_device):
    g, G = _graph("c1", cuda_device)
    args = (G.window_offset, G.original_col_indices, G.values_condensed)
    with pytest.raises(GrwsError, match="outside"):
        sample_all_layers(*args, torch.tensor([5, g.num_nodes + 40], device=cuda_device), [5],
                          g.num_nodes)
    with pytest.raises(RuntimeError, match="256"):
        sample_all_layers(*args, torch.tensor([5], device=cuda_device), [257], g.num_nodes)
    with pytest.raises(RuntimeError, match="warps_per_block"):
        sample_all_layers(*args, torch.tensor([5], device=cuda_device), [5], g.num_nodes,
                          warps_per_block=16)


def test_bcsr_sampler_layers(cuda_device):
    g, G = _graph("c1", cuda_device)
    s = BCSRSampler(fanouts=[10, 5], verbose=True)
    seeds = torch.arange(0, g.num_nodes, 11)
    layers = s.sample_layers(G, seeds)
    assert len(layers) == 2
    # layers[-1] is the hop from the seeds (drawn with fanouts[-1] = 5)
    act0 = layers[-1].active_windows.cpu().numpy()
    np.testing.assert_array_equal(act0, np.unique(seeds.numpy() // 16))
    for L in layers:
        assert L.num_rows == 16 * L.active_windows.numel()
        assert L.num_cols == g.num_nodes
        assert L.num_tiles == L.window_offset[-1].item()
    assert set(s.time_tracker) == {0, 1}
    assert "BCSRSampler" in repr(s)


@pytest.mark.parametrize("scratch", [0, 300_000])
def test_window_topk_hub_windows_without_key_scratch(cuda_device, monkeypatch, scratch):
    """Windows of more than 1,024 slots keep their keys in the caller's
    scratch (computed by the keys kernel) when it has room, and compute them
    in their own work-group (into LDS, or on every pass beyond 4,096 slots)
    when it has none (0 bytes) or runs out part-way (300 kB: some of them
    fit): the same layers either way, bit for bit against the oracle."""
    from graph_rws_amd.core import ops
    print(f"case window top-K key scratch {scratch}", flush=True)
    monkeypatch.setattr(ops, "WINDOW_KEY_SCRATCH", scratch)
    g, G = _graph("c2", cuda_device)
    seeds = synth.distinct_seeds(g.num_nodes, 1024, seed=9).numpy()
    layers, _ = sample_all_layers(G.window_offset, G.original_col_indices, G.values_condensed,
                                  torch.from_numpy(seeds).to(cuda_device), [5, 10, 15], g.num_nodes)
    ref = oracle.window_sample_all_layers(G.window_offset.cpu().numpy(), G.original_col_indices.cpu().numpy(),
                                          G.values_condensed.cpu().numpy(), seeds, [5, 10, 15], g.num_nodes)
    _compare(layers, ref)


def _layers_equal(a, b):
    assert len(a) == len(b)
    for x, y in zip(a, b):
        for u, v in zip(x, y):
            assert u.dtype == v.dtype and u.shape == v.shape
            assert torch.equal(u.cpu(), v.cpu())


@pytest.mark.parametrize("case", ["c2", "c1_hacs", "no_seeds", "minus_one_and_repeats", "bf16_tc16"])
def test_one_call_matches_the_per_layer_calls(cuda_device, case):
    """sample_all_layers runs every layer in one grws_window_sample_layers
    call (seeds from a dense per-window mask, device counts, one sync); the
    per-layer entry points (grws_window_seeds' sort, a sync per call) give
    the same layers bit for bit: full-size c2, HACS with locality, no seeds,
    seeds of -1 and repeated ids, bf16 values in 16x16 tiles."""
    from graph_rws_amd.core import ops
    print(f"case one call vs per layer {case}", flush=True)
    kw = {}
    if case == "c2":
        g, G = _graph("c2", cuda_device)
        seeds = synth.distinct_seeds(g.num_nodes, 1024, seed=21).numpy()
        fan = [5, 10, 15]
    elif case == "c1_hacs":
        g, G = _graph("c1", cuda_device)
        rng = np.random.default_rng(8)
        q = torch.from_numpy(rng.random(g.num_nodes).astype(np.float32)).to(cuda_device)
        wpart = torch.from_numpy(rng.integers(-1, 3, G.num_windows).astype(np.int32)).to(cuda_device)
        kw = dict(static_scores=q, window_part_ids=wpart,
                  part_starts=torch.tensor([0, 900, 1800], dtype=torch.int32, device=cuda_device),
                  part_ends=torch.tensor([900, 1800, 2708], dtype=torch.int32, device=cuda_device),
                  use_hacs=1, locality_enabled=1, alpha=0.5, beta=3.0, delta=0.25, gamma_bonus=0.37,
                  score_scale=250.0)
        seeds = np.arange(1, g.num_nodes, 7)
        fan = [12, 40, 3]
    elif case == "no_seeds":
        g, G = _graph("c1", cuda_device)
        seeds = np.zeros(0, np.int64)
        fan = [5, 10]
    elif case == "minus_one_and_repeats":
        g, G = _graph("c1", cuda_device)
        seeds = np.array([-1, 7, 7, 8, -1, 2700, 16, 16, 15, 0, -1])
        fan = [3, 33, 129]
    else:
        g, G = _graph("c1", cuda_device, tc=16, vdt=torch.bfloat16)
        seeds = np.arange(0, g.num_nodes, 13)
        fan = [20, 7]
    args = (G.window_offset, G.original_col_indices, G.values_condensed,
            torch.from_numpy(seeds).to(cuda_device), fan, g.num_nodes)
    tc = G.tile_cols
    one, t1 = sample_all_layers(*args, tile_cols=tc, **kw)
    per, t2 = ops._sample_all_layers_per_layer(*args, tile_cols=tc, **kw)
    _layers_equal(one, per)
    assert len(t1) == len(fan) and all(t.total_time >= 0 for t in t1)
    if case == "no_seeds":
        assert all(int(x[0][-1]) == 0 and x[3].numel() == 0 for x in one)


@pytest.mark.parametrize("path", ["one_call", "per_layer"])
def test_hacs_score_table_too_short_is_an_error(cuda_device, path):
    """A candidate column without a static score is GRWS_E_RANGE, whether
    its window is ranked by the small kernel or its keys come from the keys
    kernel (c2's windows of more than 1,024 slots), on both paths; the
    reference would read past the table."""
    from graph_rws_amd.core import ops
    print(f"case HACS short score table {path}", flush=True)
    g, G = _graph("c2", cuda_device)
    fn = sample_all_layers if path == "one_call" else ops._sample_all_layers_per_layer
    seeds = torch.arange(0, g.num_nodes, 97, device=cuda_device)
    short = torch.rand(g.num_nodes // 2, device=cuda_device)
    with pytest.raises(GrwsError, match="static score"):
        fn(G.window_offset, G.original_col_indices, G.values_condensed, seeds, [5, 10], g.num_nodes,
           static_scores=short, use_hacs=1)
    # a full table is fine, and both paths agree on it
    full = torch.rand(g.num_nodes, device=cuda_device)
    a, _ = sample_all_layers(G.window_offset, G.original_col_indices, G.values_condensed, seeds, [5, 10],
                             g.num_nodes, static_scores=full, use_hacs=1)
    b, _ = ops._sample_all_layers_per_layer(G.window_offset, G.original_col_indices, G.values_condensed, seeds,
                                            [5, 10], g.num_nodes, static_scores=full, use_hacs=1)
    _layers_equal(a, b)


def _c1_hacs(dev, G, g):
    rng = np.random.default_rng(8)
    q = torch.from_numpy(rng.random(g.num_nodes).astype(np.float32)).to(dev)
    wpart = torch.from_numpy(rng.integers(-1, 3, G.num_windows).astype(np.int32)).to(dev)
    return dict(static_scores=q, window_part_ids=wpart,
                part_starts=torch.tensor([0, 900, 1800], dtype=torch.int32, device=dev),
                part_ends=torch.tensor([900, 1800, 2708], dtype=torch.int32, device=dev),
                use_hacs=1, locality_enabled=1, alpha=0.5, beta=3.0, delta=0.25, gamma_bonus=0.37,
                score_scale=250.0)


@pytest.mark.parametrize("case", ["c2", "c1_hacs", "bf16_tc16"])
def test_captured_window_sampler_matches_the_direct_call(cuda_device, case):
    """CapturedWindowSampler (grws_window_sample_layers_enqueue captured once,
    replayed per batch, the seed count read on the device) gives the layers
    of sample_all_layers bit for bit, for batches of several seed counts
    under one capacity (the first batch runs eagerly and captures); a
    returned batch stays valid after later replays; -1, repeated and empty
    seed sets too."""
    from graph_rws_amd.core.ops import CapturedWindowSampler
    print(f"case captured window sampler {case}", flush=True)
    kw = {}
    if case == "c2":
        g, G = _graph("c2", cuda_device)
        fan, cap = [5, 10, 15], 1024
        batches = [synth.distinct_seeds(g.num_nodes, n, seed=40 + i).to(cuda_device)
                   for i, n in enumerate([1024, 1000, 1024, 513])]
    elif case == "c1_hacs":
        g, G = _graph("c1", cuda_device)
        kw = _c1_hacs(cuda_device, G, g)
        fan, cap = [12, 40, 3], 400
        batches = [torch.arange(1, g.num_nodes, 7), torch.arange(0, g.num_nodes, 9),
                   torch.tensor([-1, 7, 7, 8, -1, 16, 16, 15, 0, -1]), torch.zeros(0, dtype=torch.int64)]
    else:
        g, G = _graph("c1", cuda_device, tc=16, vdt=torch.bfloat16)
        fan, cap = [20, 7], 256
        batches = [torch.arange(0, g.num_nodes, 13), torch.arange(5, g.num_nodes, 11).to(torch.int32)]
    c = CapturedWindowSampler(G.window_offset, G.original_col_indices, G.values_condensed, fan, g.num_nodes, cap,
                              tile_cols=G.tile_cols, **kw)
    kept = []
    for i, seeds in enumerate(batches):
        got = c.run(seeds if i % 2 == 0 else seeds.cpu())
        want, _ = sample_all_layers(G.window_offset, G.original_col_indices, G.values_condensed,
                                    seeds.to(cuda_device), fan, g.num_nodes, tile_cols=G.tile_cols, **kw)
        _layers_equal(got, want)
        kept.append((got, want))
    assert c.replays == len(batches) - 1
    for got, want in kept:  # earlier batches untouched by the later replays
        _layers_equal(got, want)


def test_captured_window_sampler_errors(cuda_device):
    """An out-of-range seed is GRWS_E_RANGE after the replay and the next
    batch is fine; more seeds than the capacity are refused on the host; a
    device seed count above the capacity is clamped and flagged
    (GRWS_E_CAPACITY) by the kernel that reads the seeds."""
    from graph_rws_amd.core import ops
    from graph_rws_amd.core.ops import CapturedWindowSampler
    g, G = _graph("c1", cuda_device)
    c = CapturedWindowSampler(G.window_offset, G.original_col_indices, G.values_condensed, [5, 10], g.num_nodes,
                              64)
    good = torch.arange(0, 640, 10)
    first = c.run(good)
    with pytest.raises(GrwsError, match="outside"):
        c.run(torch.tensor([3, g.num_nodes + 5, 9]))
    _layers_equal(c.run(good), first)
    with pytest.raises(ValueError, match="capacity"):
        c.run(torch.arange(65))
    c.cnt_in.fill_(c.max_seeds + 7)
    c.graph.replay()
    torch.cuda.synchronize()
    flags = int(c.out_dev[-1].item())
    with pytest.raises(GrwsError, match="seed count"):
        ops.L.call("grws_window_sample_layers_status", flags)
    _layers_equal(c.run(good), first)


def test_bcsr_sampler_capture_option(cuda_device):
    """BCSRSampler(capture=True) samples the layers of the uncaptured
    sampler; seed counts of one bucket share a capture; modifying the
    graph's values in place makes a new one."""
    g, G = _graph("c1", cuda_device)
    a = BCSRSampler(fanouts=[10, 5], verbose=False, capture=True)
    b = BCSRSampler(fanouts=[10, 5], verbose=False)
    for n in (170, 150, 170):
        seeds = torch.arange(0, g.num_nodes, g.num_nodes // n)[:n]
        for x, y in zip(a.sample_layers(G, seeds), b.sample_layers(G, seeds)):
            for name in ("window_offset", "original_col_indices", "values_condensed", "active_windows",
                         "active_masks"):
                assert torch.equal(getattr(x, name).cpu(), getattr(y, name).cpu()), name
            assert (x.num_rows, x.num_cols) == (y.num_rows, y.num_cols)
    assert len(a._captures) == 1
    cap = next(iter(a._captures.values()))[1]
    assert cap.replays == 2
    G.values_condensed.mul_(0.5)
    seeds = torch.arange(0, g.num_nodes, 17)
    for x, y in zip(a.sample_layers(G, seeds), b.sample_layers(G, seeds)):
        assert torch.equal(x.values_condensed.cpu(), y.values_condensed.cpu())
    assert next(iter(a._captures.values()))[1] is not cap
