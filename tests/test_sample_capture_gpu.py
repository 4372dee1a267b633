"""Captured sampling (grws_sample_blocks_enqueue replayed from a HIP graph,
NeighborSampler(capture=True)): every batch equals the uncaptured call bit
for bit, including the transposed blocks; seed counts of one bucket share a
capture (the count is read on the device); a returned batch stays valid
after later replays (its tensors are copies); errors flagged on the device
raise after the replay and leave the state clean."""
import numpy as np
import pytest
import torch

import oracle
from graph_rws_amd import synth
from graph_rws_amd.core._lib import GrwsError
from graph_rws_amd.core.ops import CapturedSampleBlocks, SampleState, sample_blocks
from graph_rws_amd.sampler import NeighborSampler

pytestmark = pytest.mark.gpu


def _same_batch(a, b):
    assert len(a) == len(b)
    for h, (x, y) in enumerate(zip(a, b)):
        assert len(x) == len(y)
        for i, (u, v) in enumerate(zip(x, y)):
            if isinstance(u, torch.Tensor):
                assert u.dtype == v.dtype and u.shape == v.shape, f"hop {h} item {i}"
                assert torch.equal(u.view(torch.uint8) if u.element_size() == 2 else u,
                                   v.view(torch.uint8) if v.element_size() == 2 else v), f"hop {h} item {i}"
            elif isinstance(u, tuple):
                _same_batch([u], [v])
            else:
                assert u == v, f"hop {h} item {i}"


@pytest.mark.parametrize("vdt,tc,thops", [(torch.float16, 16, [True, True, False]),
                                          (torch.float32, 8, None),
                                          (torch.bfloat16, 16, [False, True, True])])
def test_captured_batches_equal_the_direct_call(cuda_device, vdt, tc, thops):
    print(f"case captured sampling {vdt} tc={tc} transposes={thops}", flush=True)
    g = synth.c5_graph(device=cuda_device, scale=2e-4)
    st = SampleState(g.num_nodes, cuda_device)
    hops = [5, 10, 15]
    cap = CapturedSampleBlocks(g.row_ptr, g.col_idx, hops, st, 42, tc, vdt, thops, 320)
    kept = []
    for i, n in enumerate([300, 320, 257, 320, 1, 300]):
        seeds = synth.distinct_seeds(g.num_nodes, n, seed=100 + i, device=cuda_device)
        got = cap.run(seeds if i % 2 else seeds.cpu())
        want = sample_blocks(g.row_ptr, g.col_idx, seeds, hops, st, seed=42, tile_cols=tc, values_dtype=vdt,
                             transposes=thops)
        _same_batch(got, want)
        kept.append((got, want))
        assert bool((st.node_map == -1).all()) and bool((st.bitmap == 0).all())
    assert cap.replays == 5
    for got, want in kept:  # earlier batches untouched by the later replays
        _same_batch(got, want)


def test_captured_seeds_of_any_layout(cuda_device):
    """The captured call stages contiguous int64 device seeds with one copy
    launch and any other seeds through torch's copy: a strided view, int32
    seeds, a 2-D seed tensor and host seeds all give the batch of the same
    seeds passed contiguous."""
    print("case captured sampling seed layouts", flush=True)
    g = synth.c5_graph(device=cuda_device, scale=2e-4)
    st = SampleState(g.num_nodes, cuda_device)
    hops = [5, 10, 15]
    cap = CapturedSampleBlocks(g.row_ptr, g.col_idx, hops, st, 42, 16, torch.float16, None, 256)
    base = synth.distinct_seeds(g.num_nodes, 512, seed=7, device=cuda_device)
    seeds = base[::2].clone()  # 256 seeds, contiguous
    want = cap.run(seeds)
    pad = torch.stack([seeds, base[1::2]], 1).contiguous()  # seeds at stride 2, 16-byte aligned
    for variant in (pad[:, 0], seeds.to(torch.int32), seeds.view(16, 16), seeds.cpu()):
        _same_batch(cap.run(variant), want)


def test_neighbor_sampler_capture_matches_oracle(cuda_device):
    """The sampler with capture=True, batches of one bucket and of another,
    against the oracle; the captures are reused."""
    print("case neighbor sampler capture", flush=True)
    g = synth.c5_graph(device=cuda_device, scale=2e-4)
    s = NeighborSampler([15, 10, 5], seed=42, tile_cols=16, values_dtype=torch.float16, capture=True)
    ip, ix = g.row_ptr.cpu().numpy(), g.col_idx.cpu().numpy()
    for i, n in enumerate([256, 250, 256, 300, 256]):
        seeds = synth.distinct_seeds(g.num_nodes, n, seed=7 + i, device=cuda_device)
        blocks = s.sample_layers(g.row_ptr, g.col_idx, seeds, transposes=[False, True, True])
        ref = oracle.sample_blocks(ip, ix, seeds.cpu().numpy(), [15, 10, 5], seed=42, tile_cols=16)
        for b, r in zip(blocks, ref):
            np.testing.assert_array_equal(b.src_nodes.cpu().numpy(), r["src_nodes"])
            np.testing.assert_array_equal(b.window_offset.cpu().numpy(), r["win"])
            np.testing.assert_array_equal(b.original_col_indices.cpu().numpy(), r["cols"])
            assert torch.equal(b.values_condensed.cpu(), torch.from_numpy(r["vals"]).half())
        from graph_rws_amd import builder
        for b in blocks[1:]:
            AT, fresh = b.transpose(), builder.transpose(b)
            assert torch.equal(AT.original_col_indices, fresh.original_col_indices)
            assert torch.equal(AT.values_condensed, fresh.values_condensed)
    assert len(s._captures) == 2  # buckets of 256 and 320 seeds
    assert sum(c.replays for c in s._captures.values()) == 3


def test_captured_batch_errors(cuda_device):
    """Duplicate seeds and a count above the capacity are flagged on the
    device and raised after the replay; the state stays clean and the next
    batch is right."""
    print("case captured sampling errors", flush=True)
    g = synth.c5_graph(device=cuda_device, scale=1e-4)
    st = SampleState(g.num_nodes, cuda_device)
    cap = CapturedSampleBlocks(g.row_ptr, g.col_idx, [3, 3], st, 42, 16, torch.float32, None, 64)
    good = synth.distinct_seeds(g.num_nodes, 50, seed=1, device=cuda_device)
    cap.run(good)  # eager + capture
    dup = good.clone()
    dup[7] = dup[3]
    with pytest.raises(GrwsError, match="twice"):
        cap.run(dup)  # replayed
    assert bool((st.node_map == -1).all()) and bool((st.bitmap == 0).all())
    with pytest.raises(ValueError, match="capacity"):
        cap.run(torch.arange(65, device=cuda_device))
    _same_batch(cap.run(good), sample_blocks(g.row_ptr, g.col_idx, good, [3, 3], st, seed=42, tile_cols=16))
