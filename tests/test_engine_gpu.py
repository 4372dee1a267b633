"""Mini-batch training on the GPU (helper/engine.py:86-256 of the reference):
one NeighborSampler batch through GCN_BCSR against a float64 dense
restatement of the same blocks, and full epochs of both samplers through
train_epoch_node_sampling (pipelined and serial)."""
import copy

import numpy as np
import pytest
import torch

import oracle
from graph_rws_amd import synth
from graph_rws_amd.data import BCSRGraph
from graph_rws_amd.helper import EpochTimer, train_epoch_node_sampling
from graph_rws_amd.models import GCN_BCSR
from graph_rws_amd.sampler import BCSRSampler, NeighborSampler

pytestmark = pytest.mark.gpu


def test_block_step_matches_dense_reference(cuda_device):
    """Loss and every gradient of one mini-batch step (fp32) equal float64
    autograd over dense copies of the sampled blocks (tolerance 1e-4 of the
    largest magnitude)."""
    print("case block step", flush=True)
    torch.manual_seed(0)
    g = synth.c5_graph(device=cuda_device, scale=1e-4)
    seeds = synth.distinct_seeds(g.num_nodes, 64, seed=3, device=cuda_device)
    blocks = NeighborSampler([6, 4, 3]).sample_layers(g.row_ptr, g.col_idx, seeds)
    X = synth.features(g.num_nodes, 32, seed=4, device=cuda_device)
    labels = torch.randint(0, 5, (g.num_nodes,), device=cuda_device)
    model = GCN_BCSR(32, 24, 5, 3, dropout=0.0, use_checkpoint=False).to(cuda_device)
    ref = copy.deepcopy(model).cpu().double()
    dense = [torch.from_numpy(oracle.bcsr_to_dense(b.window_offset.cpu().numpy(),
                                                   b.original_col_indices.cpu().numpy(),
                                                   b.values_condensed.cpu().numpy(), 16,
                                                   b.tile_cols, b.num_cols)[:b.num_rows])
             for b in blocks]
    feats = X.index_select(0, blocks[0].src_nodes)
    logits = model(blocks, feats)
    assert logits.shape == (64, 5)
    loss = torch.nn.functional.cross_entropy(logits, labels[seeds])
    loss.backward()

    h = feats.double().cpu()
    for l, (layer, A) in enumerate(zip(ref.layers, dense)):
        h = A @ (h @ layer.weight_neigh) + h[: A.shape[0]] @ layer.weight_self
        if l < 2:
            h = ref.norms[l](torch.relu(h))
    rl = torch.nn.functional.cross_entropy(h, labels[seeds].cpu())
    rl.backward()
    assert abs(float(loss) - float(rl)) <= 1e-4 * abs(float(rl))
    for (n, p), (_, q) in zip(model.named_parameters(), ref.named_parameters()):
        a, b = p.grad.double().cpu(), q.grad
        assert float((a - b).abs().max()) <= 1e-4 * max(float(b.abs().max()), 1e-30), n


@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_block_step_c5_widths(cuda_device, dt):
    """One mini-batch step at c5's configured shape: 1,024 seeds, fanouts
    [15, 10, 5] (Philox seed 42), 128 -> 256 -> 256 -> 172, on a c5 graph
    at 1e-3 scale (111k nodes, 1.6M edges), against float64 autograd over
    dense copies of the same blocks and features (/root/reference/helper/
    engine.py:86-256 through models/model.py:212-266).

    The reference applies the device's ReLU masks (a unit within rounding
    of zero may take the other sign in float64 and pass or drop its whole
    gradient: with its own masks the float32 gradients of layers 0-1 were
    3e-4 off, the float16 ones 2%).

    float32 (block values and features float32, no autocast): the loss
    within 1e-4 relative, every gradient within 2e-5 relative in the
    Frobenius norm and within 5e-5 of its largest magnitude elementwise
    (measured: 4e-6 at worst).  float16 (float16 block values and
    features, float16 autocast, as c5 runs): autocast rounds every GEMM
    and SpMM output to float16 (u = 2^-11 = 4.9e-4) through three layers,
    LayerNorm and the backward pass: the loss within 1e-2 relative, every
    gradient within 1e-2 relative in the Frobenius norm and within 1e-2 of
    its largest magnitude elementwise (measured: 2.8e-3 at worst, a few
    float16 roundings)."""
    print(f"case block step c5 widths {dt}", flush=True)
    torch.manual_seed(0)
    dev = cuda_device
    g = synth.c5_graph(device=dev, scale=1e-3)
    seeds = synth.distinct_seeds(g.num_nodes, 1024, seed=3, device=dev)
    blocks = NeighborSampler([15, 10, 5], seed=42, values_dtype=dt).sample_layers(g.row_ptr, g.col_idx, seeds)
    assert [b.num_rows for b in blocks][-1] == 1024
    X = synth.features(g.num_nodes, 128, seed=4, device=dev).to(dt)
    labels = torch.randint(0, 172, (g.num_nodes,), device=dev)
    model = GCN_BCSR(128, 256, 172, 3, dropout=0.0, use_checkpoint=False).to(dev)
    ref = copy.deepcopy(model).cpu().double()
    dense = [torch.from_numpy(oracle.bcsr_to_dense(b.window_offset.cpu().numpy(),
                                                   b.original_col_indices.cpu().numpy(),
                                                   b.values_condensed.float().cpu().numpy(), 16,
                                                   b.tile_cols, b.num_cols)[:b.num_rows]).double()
             for b in blocks]
    feats = X.index_select(0, blocks[0].src_nodes)
    # the device's ReLU masks (each hidden layer's output > 0, taken where
    # the fused ReLU + LayerNorm tail receives it): the reference applies
    # them instead of its own, so that activations within rounding of zero,
    # whose sign the two sides may see differently, do not move the
    # comparison (a flipped unit passes or drops a whole gradient)
    masks = []
    tail = model._hidden_tail

    def spy(l, h, training):
        masks.append((h > 0).detach().cpu())
        return tail(l, h, training)

    model._hidden_tail = spy
    with torch.autocast("cuda", dtype=torch.float16, enabled=dt == torch.float16):
        logits = model(blocks, feats)
    del model._hidden_tail
    assert logits.shape == (1024, 172) and len(masks) == 2
    loss = torch.nn.functional.cross_entropy(logits.float(), labels[seeds])
    loss.backward()

    h = feats.double().cpu()
    for l, (layer, A) in enumerate(zip(ref.layers, dense)):
        h = A @ (h @ layer.weight_neigh) + h[: A.shape[0]] @ layer.weight_self
        if l < 2:
            flips = int(((h > 0) != masks[l]).sum())
            print(f"layer {l}: {flips} of {h.numel()} ReLU signs differ from the device's", flush=True)
            h = ref.norms[l](h * masks[l])
    rl = torch.nn.functional.cross_entropy(h, labels[seeds].cpu())
    rl.backward()
    f16 = dt == torch.float16
    assert abs(float(loss) - float(rl)) <= (1e-2 if f16 else 1e-4) * abs(float(rl)), (float(loss), float(rl))
    fro_tol, max_tol = (1e-2, 1e-2) if f16 else (2e-5, 5e-5)
    bad = []
    for (n, p), (_, q) in zip(model.named_parameters(), ref.named_parameters()):
        a, b = p.grad.double().cpu(), q.grad
        fro = float((a - b).norm()) / max(float(b.norm()), 1e-30)
        mx = float((a - b).abs().max()) / max(float(b.abs().max()), 1e-30)
        print(f"{n}: error / largest {mx:.3e}, Frobenius {fro:.3e}", flush=True)
        if fro > fro_tol or mx > max_tol:
            bad.append((n, fro, mx))
    assert not bad, bad


@pytest.mark.parametrize("pipeline", [True, False])
def test_neighbor_sampler_epoch(cuda_device, pipeline):
    print(f"case neighbor epoch pipeline={pipeline}", flush=True)
    torch.manual_seed(1)
    g = synth.c5_graph(device=cuda_device, scale=2e-4)
    X = synth.features(g.num_nodes, 64, seed=5, device=cuda_device).half()
    labels = X[:, :4].float().argmax(1)  # a function of each node's own features
    train_idx = torch.arange(0, g.num_nodes, 4)
    model = GCN_BCSR(64, 64, 4, 3, dropout=0.0, use_checkpoint=False).to(cuda_device)
    opt = torch.optim.Adam(model.parameters(), lr=0.01)
    sampler = NeighborSampler([10, 5, 5], values_dtype=torch.float16)
    timer = EpochTimer()
    losses = []
    for _ in range(4):
        with torch.autocast("cuda", dtype=torch.float16):
            loss, acc = train_epoch_node_sampling(model, g, X, labels, train_idx, opt,
                                                  cuda_device, sampler, batch_size=512,
                                                  timer=timer, pipeline=pipeline)
        losses.append(loss)
    assert all(np.isfinite(losses)), losses
    assert losses[-1] < losses[0], losses
    st = timer.get_epoch_stats()
    assert set(st) >= {"Data", "Sample", "Fwd", "Bwd", "Step", "SpMM"}


@pytest.mark.parametrize("pipeline", [True, False])
def test_window_sampler_epoch(cuda_device, pipeline):
    """The reference's own mini-batch path: BCSRSampler layers over the full
    BCSR graph, reindex_bcsr between layers, seed rows found through the
    active windows."""
    print(f"case window epoch pipeline={pipeline}", flush=True)
    torch.manual_seed(2)
    g = synth.config_graph("c1")
    G = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes,
                           tile_cols=8, device=cuda_device)
    X = synth.features(g.num_nodes, 1433, kind="binary", seed=2, device=cuda_device)
    R = torch.randn(1433, 7, generator=torch.Generator().manual_seed(3)).to(cuda_device)
    labels = (X @ R).argmax(1)  # learnable through the self path
    train_idx = torch.arange(g.num_nodes)
    model = GCN_BCSR(1433, 32, 7, 2, dropout=0.0, use_checkpoint=False).to(cuda_device)
    opt = torch.optim.Adam(model.parameters(), lr=0.01)
    sampler = BCSRSampler(fanouts=[10, 10], verbose=False)
    losses = [train_epoch_node_sampling(model, G, X, labels, train_idx, opt, cuda_device, sampler,
                                        batch_size=256, pipeline=pipeline)[0] for _ in range(4)]
    assert all(np.isfinite(losses)), losses
    assert losses[-1] < losses[0], losses
