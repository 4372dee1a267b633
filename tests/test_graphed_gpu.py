"""GraphedFullStep: the full-graph training step captured once on a HIP
graph and replayed.

* With dropout off, every replay leaves the parameters equal to those of an
  eager twin that ran the same number of steps (same kernels on the same
  values); eager work and a synchronisation run between replays, and every
  replay is checked, so a graph node that replays wrongly after the first
  replay fails here.
* With dropout on, each replay draws a new mask (the seed is drawn on the
  device inside the graph), and the kept elements carry exactly the
  undropped values times 1/(1-p).
"""
import copy

import pytest
import torch

from graph_rws_amd import synth
from graph_rws_amd.data import BCSRGraph
from graph_rws_amd.helper import GraphedFullStep, train_epoch_full
from graph_rws_amd.layers.fused import act_norm_dropout
from graph_rws_amd.models import GCN_BCSR

pytestmark = pytest.mark.gpu


def _setup(dev, cfg, dt):
    g = synth.config_graph(cfg, device=dev, scale=1.0 if cfg == "c1" else 0.02)
    vdt = torch.float32 if dt is None else dt
    G = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes, tile_cols=16,
                           device=dev, values_dtype=vdt)
    d = 1433 if cfg == "c1" else 608
    X = synth.features(g.num_nodes, d, seed=5, device=dev, kind="binary" if cfg == "c1" else "normal")
    if dt is not None:
        X = X.to(dt)
    gen = torch.Generator(device=dev)
    gen.manual_seed(6)
    classes = 7 if cfg == "c1" else 41
    labels = torch.randint(0, classes, (g.num_nodes,), generator=gen, device=dev)
    train_idx = torch.nonzero(torch.rand(g.num_nodes, generator=gen, device=dev) < 0.5).view(-1)
    return G, X, labels, train_idx, d, classes


@pytest.mark.parametrize("cfg,dt", [("c1", None), ("c3", torch.float16)])
def test_graphed_step_tracks_eager(cuda_device, cfg, dt):
    print(f"case graphed-vs-eager {cfg} {dt}", flush=True)
    dev = cuda_device
    G, X, labels, train_idx, d, classes = _setup(dev, cfg, dt)
    hidden, layers = (16, 2) if cfg == "c1" else (64, 3)
    torch.manual_seed(7)
    m_e = GCN_BCSR(d, hidden, classes, layers, dropout=0.0, use_checkpoint=False).to(dev)
    m_g = copy.deepcopy(m_e)
    o_e = torch.optim.Adam(m_e.parameters(), lr=0.01, capturable=True)
    o_g = torch.optim.Adam(m_g.parameters(), lr=0.01, capturable=True)

    def eager():
        if dt is None:
            return train_epoch_full(m_e, G, X, labels, train_idx, o_e, dev, sync=False)
        with torch.autocast("cuda", dtype=dt):
            return train_epoch_full(m_e, G, X, labels, train_idx, o_e, dev, sync=False)

    warm = 3
    step = GraphedFullStep(m_g, G, X, labels, train_idx, o_g, dev, warmup=warm, autocast_dtype=dt)
    for _ in range(warm):
        eager()
    for r in range(4):
        loss_g, _ = step()
        loss_e, _ = eager()
        torch.cuda.synchronize()
        assert torch.isfinite(loss_g).all()
        torch.testing.assert_close(loss_g, loss_e, rtol=1e-5, atol=1e-6, msg=f"replay {r}: loss")
        for (n, p), (_, q) in zip(m_g.named_parameters(), m_e.named_parameters()):
            torch.testing.assert_close(p, q, rtol=1e-5, atol=1e-6, msg=f"replay {r}: {n}")


def test_graphed_dropout_draws_new_mask_each_replay(cuda_device):
    print("case graphed dropout", flush=True)
    dev = cuda_device
    torch.manual_seed(8)
    z = torch.randn(300, 64, device=dev)
    norm = torch.nn.LayerNorm(64).to(dev)
    with torch.no_grad():
        ref = act_norm_dropout(z, norm, 0.0, True)           # no dropout: the kept values / (1 - p)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side), torch.no_grad():
        act_norm_dropout(z, norm, 0.5, True)
    torch.cuda.current_stream(dev).wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.graph(g):
        out = act_norm_dropout(z, norm, 0.5, True)
    masks = []
    for r in range(3):
        g.replay()
        torch.cuda.synchronize()
        kept = out != 0
        frac = float(kept.float().mean())
        assert 0.4 < frac < 0.6, frac
        assert torch.equal(out[kept], (ref * 2.0)[kept]), f"replay {r}"
        masks.append(kept.clone())
        torch.randn(1000, device=dev).sum()                  # eager work between replays
    assert not torch.equal(masks[0], masks[1]) and not torch.equal(masks[1], masks[2])


def test_graphed_step_reads_features_updated_in_place(cuda_device):
    """c4's layer 0 gathers its 112 bf16 features through a line-aligned,
    zero-padded copy.  Under capture that copy must be made inside the graph,
    so a replay after features.copy_(new) trains on the new values: each
    replay is checked against an eager twin fed the same features."""
    print("case graphed features copy_ (c4 shape, 1%, bf16)", flush=True)
    dev = cuda_device
    g = synth.config_graph("c4", device=dev, scale=0.01)
    G = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes, tile_cols=16,
                           device=dev, values_dtype=torch.bfloat16)
    X = synth.features(g.num_nodes, 112, seed=5, device=dev).to(torch.bfloat16)
    assert G.padded_input(X) is not None, "the case must gather through the aligned copy"
    gen = torch.Generator(device=dev)
    gen.manual_seed(6)
    labels = torch.randint(0, 47, (g.num_nodes,), generator=gen, device=dev)
    train_idx = torch.nonzero(torch.rand(g.num_nodes, generator=gen, device=dev) < 0.5).view(-1)
    torch.manual_seed(7)
    m_e = GCN_BCSR(112, 64, 47, 3, dropout=0.0, use_checkpoint=False).to(dev)
    m_g = copy.deepcopy(m_e)
    o_e = torch.optim.Adam(m_e.parameters(), lr=0.01, capturable=True)
    o_g = torch.optim.Adam(m_g.parameters(), lr=0.01, capturable=True)

    def eager():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            return train_epoch_full(m_e, G, X, labels, train_idx, o_e, dev, sync=False)

    warm = 3
    step = GraphedFullStep(m_g, G, X, labels, train_idx, o_g, dev, warmup=warm, autocast_dtype=torch.bfloat16)
    for _ in range(warm):
        eager()
    for r in range(3):
        X.copy_(synth.features(g.num_nodes, 112, seed=100 + r, device=dev).to(torch.bfloat16))
        loss_g, _ = step()
        loss_e, _ = eager()
        torch.cuda.synchronize()
        torch.testing.assert_close(loss_g, loss_e, rtol=1e-5, atol=1e-6, msg=f"replay {r}: loss")
        for (n, p), (_, q) in zip(m_g.named_parameters(), m_e.named_parameters()):
            torch.testing.assert_close(p, q, rtol=1e-5, atol=1e-6, msg=f"replay {r}: {n}")
