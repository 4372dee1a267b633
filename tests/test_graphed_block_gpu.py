"""GraphedBlockStep: the node-wise mini-batch step captured per bucket of
batch shapes on a HIP graph and replayed, against the eager step.

The bucket pads every block to a round row count; the padded rows have no
neighbours and no loss, so each replay must train as the eager step does on
the same batch.  GEMMs over the padded shapes may reduce in another order,
so the comparison carries a tolerance (stated per dtype below) instead of
bit equality.  Adam's eps is raised to 1.0 on both sides, which makes each
update about lr * gradient: at eps 1e-8 an entry's update is about
lr * sign(gradient), and near eps an update moves lr / eps per unit of
gradient, so rounding differences of a near-zero gradient entry would be
amplified into parameter differences of order lr.
"""
import copy

import numpy as np
import pytest
import torch

from graph_rws_amd import synth
from graph_rws_amd.helper import EpochTimer, GraphedBlockStep, train_epoch_node_sampling
from graph_rws_amd.helper.engine import loss_and_metrics_rows
from graph_rws_amd.models import GCN_BCSR
from graph_rws_amd.sampler import NeighborSampler

pytestmark = pytest.mark.gpu

# (loss rtol, parameter atol) after each step: float32, float16 autocast
TOL = {None: (1e-4, 2e-5), torch.float16: (1e-2, 5e-4)}


def _eager_step(model, opt, blocks, feats, labels, dt):
    model.train()
    opt.zero_grad()
    with torch.autocast("cuda", dtype=dt or torch.float16, enabled=dt is not None):
        logits = model(blocks, feats)
    loss, correct, _ = loss_and_metrics_rows(logits, None, labels, check_rows=False)
    loss.backward()
    torch.nn.utils.clip_grad_norm_(model.parameters(), max_norm=1.0)
    opt.step()
    return loss.detach(), correct


@pytest.mark.parametrize("dt,tc", [(None, 16), (torch.float16, 16), (None, 8)])
def test_graphed_block_step_tracks_eager(cuda_device, dt, tc):
    print(f"case graphed block step dtype={dt} tile_cols={tc}", flush=True)
    dev = cuda_device
    g = synth.c5_graph(device=dev, scale=1e-4)
    D = 48
    X = synth.features(g.num_nodes, D, seed=4, device=dev)
    vdt = torch.float32
    if dt is not None:
        X, vdt = X.to(dt), dt
    labels = X[:, :5].float().argmax(1)
    torch.manual_seed(7)
    m_e = GCN_BCSR(D, 32, 5, 3, dropout=0.0, use_checkpoint=False).to(dev)
    m_g = copy.deepcopy(m_e)
    o_e = torch.optim.Adam(m_e.parameters(), lr=0.01, eps=1.0, capturable=True)
    o_g = torch.optim.Adam(m_g.parameters(), lr=0.01, eps=1.0, capturable=True)
    step = GraphedBlockStep(m_g, o_g, dev, autocast_dtype=dt, warmup=2)
    sampler = NeighborSampler([6, 4, 3], tile_cols=tc, values_dtype=vdt)
    rtol, atol = TOL[dt]
    sizes = [200, 230, 200, 64, 230, 200]
    for b, n in enumerate(sizes):
        seeds = torch.sort(synth.distinct_seeds(g.num_nodes, n, seed=10 + b, device=dev)).values
        blocks = sampler.sample_layers(g.row_ptr, g.col_idx, seeds)
        feats = X.index_select(0, blocks[0].src_nodes)
        lab = labels[seeds]
        loss_g, corr_g = step(blocks, feats, lab)
        loss_g, corr_g = loss_g.clone(), corr_g.clone()
        loss_e, corr_e = _eager_step(m_e, o_e, blocks, feats, lab, dt)
        torch.cuda.synchronize()
        assert torch.isfinite(loss_g).all()
        torch.testing.assert_close(loss_g.float(), loss_e.float(), rtol=rtol, atol=rtol,
                                   msg=f"batch {b}: loss")
        assert abs(int(corr_g) - int(corr_e)) <= max(1, n // 100), (b, int(corr_g), int(corr_e))
        for (name, p), (_, q) in zip(m_g.named_parameters(), m_e.named_parameters()):
            torch.testing.assert_close(p, q, rtol=0, atol=atol, msg=f"batch {b}: {name}")
    # at least two buckets (64 seeds vs 200-230), and some batch replays a
    # bucket captured before it
    assert 2 <= step.captures < len(sizes), step.captures
    assert len(step.buckets) == step.captures


def test_graphed_block_step_c5_widths(cuda_device):
    """The captured step at c5's configured widths (128 -> 256 -> 256 ->
    172, float16 autocast, fanouts [15, 10, 5], about 1,024 seeds per
    batch, c5 graph at 1e-3 scale) tracks the eager step batch by batch."""
    print("case graphed block step c5 widths", flush=True)
    dev = cuda_device
    g = synth.c5_graph(device=dev, scale=1e-3)
    X = synth.features(g.num_nodes, 128, seed=4, device=dev).half()
    labels = X.float().argmax(1)  # 128 of the 172 classes occur
    torch.manual_seed(7)
    m_e = GCN_BCSR(128, 256, 172, 3, dropout=0.0, use_checkpoint=False).to(dev)
    m_g = copy.deepcopy(m_e)
    o_e = torch.optim.Adam(m_e.parameters(), lr=0.01, eps=1.0, capturable=True)
    o_g = torch.optim.Adam(m_g.parameters(), lr=0.01, eps=1.0, capturable=True)
    step = GraphedBlockStep(m_g, o_g, dev, autocast_dtype=torch.float16, warmup=2)
    sampler = NeighborSampler([15, 10, 5], seed=42, values_dtype=torch.float16)
    rtol, atol = TOL[torch.float16]
    for b, n in enumerate([1024, 1024, 1000, 1024]):
        seeds = torch.sort(synth.distinct_seeds(g.num_nodes, n, seed=20 + b, device=dev)).values
        blocks = sampler.sample_layers(g.row_ptr, g.col_idx, seeds)
        feats = X.index_select(0, blocks[0].src_nodes)
        lab = labels[seeds]
        loss_g, corr_g = step(blocks, feats, lab)
        loss_g, corr_g = loss_g.clone(), corr_g.clone()
        loss_e, corr_e = _eager_step(m_e, o_e, blocks, feats, lab, torch.float16)
        torch.cuda.synchronize()
        assert torch.isfinite(loss_g).all()
        torch.testing.assert_close(loss_g.float(), loss_e.float(), rtol=rtol, atol=rtol, msg=f"batch {b}: loss")
        assert abs(int(corr_g) - int(corr_e)) <= max(1, n // 100), (b, int(corr_g), int(corr_e))
        for (name, p), (_, q) in zip(m_g.named_parameters(), m_e.named_parameters()):
            torch.testing.assert_close(p, q, rtol=0, atol=atol, msg=f"batch {b}: {name}")
    assert step.captures >= 1


def test_capture_while_another_thread_samples(cuda_device):
    """A bucket is captured while another thread samples on its own stream
    (stream syncs, device-to-host copies, allocations), as the pipelined
    epoch's producer does when a new batch shape appears mid-epoch: the
    capture is thread-local, so neither thread's work fails, and the
    replayed step still tracks the eager one."""
    import threading
    print("case capture while another thread samples", flush=True)
    dev = cuda_device
    g = synth.c5_graph(device=dev, scale=2e-4)
    D = 48
    X = synth.features(g.num_nodes, D, seed=4, device=dev).half()
    labels = X[:, :5].float().argmax(1)
    torch.manual_seed(3)
    m_e = GCN_BCSR(D, 32, 5, 3, dropout=0.0, use_checkpoint=False).to(dev)
    m_g = copy.deepcopy(m_e)
    o_e = torch.optim.Adam(m_e.parameters(), lr=0.01, eps=1.0, capturable=True)
    o_g = torch.optim.Adam(m_g.parameters(), lr=0.01, eps=1.0, capturable=True)
    step = GraphedBlockStep(m_g, o_g, dev, autocast_dtype=torch.float16, warmup=2)
    main_sampler = NeighborSampler([6, 4, 3], values_dtype=torch.float16)
    stop, started, failures, done = threading.Event(), threading.Event(), [], [0]

    def producer():
        try:
            s = torch.cuda.Stream(device=dev)
            smp = NeighborSampler([6, 4, 3], values_dtype=torch.float16)
            with torch.cuda.stream(s):
                i = 0
                while not stop.is_set() and i < 2000:
                    sd = synth.distinct_seeds(g.num_nodes, 150 + (i % 7), seed=500 + i, device=dev)
                    bl = smp.sample_layers(g.row_ptr, g.col_idx, sd)
                    int(bl[0].src_nodes.numel())
                    bl[-1].window_offset.cpu()
                    s.synchronize()
                    i += 1
                    done[0] = i
                    started.set()
        except BaseException as e:  # reported by the main thread
            failures.append(e)
            started.set()

    th = threading.Thread(target=producer)
    th.start()
    try:
        assert started.wait(120), "the producer thread did not start"
        rtol, atol = TOL[torch.float16]
        for b, n in enumerate([200, 64, 200, 64]):
            seeds = torch.sort(synth.distinct_seeds(g.num_nodes, n, seed=30 + b, device=dev)).values
            blocks = main_sampler.sample_layers(g.row_ptr, g.col_idx, seeds)
            feats = X.index_select(0, blocks[0].src_nodes)
            lab = labels[seeds]
            loss_g, _ = step(blocks, feats, lab)
            loss_g = loss_g.clone()
            loss_e, _ = _eager_step(m_e, o_e, blocks, feats, lab, torch.float16)
            torch.cuda.synchronize()
            torch.testing.assert_close(loss_g.float(), loss_e.float(), rtol=rtol, atol=rtol, msg=f"batch {b}")
    finally:
        stop.set()
        th.join(timeout=120)
    assert not th.is_alive(), "the producer thread did not finish"
    assert not failures, failures
    assert step.captures == 2 and done[0] > 0


def test_graphed_block_epoch(cuda_device):
    """train_epoch_node_sampling with graphed=: the pipelined epoch replays
    captured steps and trains like the eager epoch (dropout off)."""
    print("case graphed block epoch", flush=True)
    dev = cuda_device
    g = synth.c5_graph(device=dev, scale=2e-4)
    X = synth.features(g.num_nodes, 64, seed=5, device=dev).half()
    labels = X[:, :4].float().argmax(1)
    train_idx = torch.arange(0, g.num_nodes, 4)
    torch.manual_seed(1)
    m_e = GCN_BCSR(64, 64, 4, 3, dropout=0.0, use_checkpoint=False).to(dev)
    m_g = copy.deepcopy(m_e)
    o_e = torch.optim.Adam(m_e.parameters(), lr=0.3, eps=1.0, capturable=True)
    o_g = torch.optim.Adam(m_g.parameters(), lr=0.3, eps=1.0, capturable=True)
    step = GraphedBlockStep(m_g, o_g, dev, autocast_dtype=torch.float16)
    s_e = NeighborSampler([10, 5, 5], values_dtype=torch.float16)
    s_g = NeighborSampler([10, 5, 5], values_dtype=torch.float16)
    le, lg = [], []
    for _ in range(3):
        timer = EpochTimer()
        with torch.autocast("cuda", dtype=torch.float16):
            lg.append(train_epoch_node_sampling(m_g, g, X, labels, train_idx, o_g, dev, s_g, batch_size=512,
                                                timer=timer, pipeline=True, graphed=step)[0])
            le.append(train_epoch_node_sampling(m_e, g, X, labels, train_idx, o_e, dev, s_e, batch_size=512,
                                                pipeline=True)[0])
    assert all(np.isfinite(lg)), lg
    assert lg[-1] < lg[0], lg
    np.testing.assert_allclose(lg, le, rtol=2e-2)
    assert timer.get_epoch_stats()["Step"] > 0
    assert 1 <= step.captures <= 6, step.captures


def test_graphed_block_dropout_new_mask_each_replay(cuda_device):
    """With dropout on, two replays of one batch from the same parameters
    draw different masks (the seed is drawn on the device in the graph)."""
    print("case graphed block dropout", flush=True)
    dev = cuda_device
    g = synth.c5_graph(device=dev, scale=1e-4)
    X = synth.features(g.num_nodes, 32, seed=4, device=dev)
    labels = X[:, :3].argmax(1)
    torch.manual_seed(3)
    m = GCN_BCSR(32, 64, 3, 2, dropout=0.5, use_checkpoint=False).to(dev)
    o = torch.optim.Adam(m.parameters(), lr=0.0, capturable=True)  # lr 0: parameters stay put
    step = GraphedBlockStep(m, o, dev)
    seeds = torch.sort(synth.distinct_seeds(g.num_nodes, 300, seed=9, device=dev)).values
    blocks = NeighborSampler([5, 5]).sample_layers(g.row_ptr, g.col_idx, seeds)
    feats = X.index_select(0, blocks[0].src_nodes)
    l1 = step(blocks, feats, labels[seeds])[0].clone()
    l2 = step(blocks, feats, labels[seeds])[0].clone()
    torch.cuda.synchronize()
    assert torch.isfinite(l1) and torch.isfinite(l2)
    assert float(l1) != float(l2)
    assert step.captures == 1
