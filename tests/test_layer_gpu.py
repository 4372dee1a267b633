"""BCSRSPMMFunction / BCSRGraphConv / GCN_BCSR on the GPU against a float64
dense restatement of the reference model (layers/layer.py:28-191,
models/model.py:212-266) on the CPU, with the same parameters.

Tolerances: float32 end to end |d| <= 1e-4 * scale (the GEMMs run in fp32
on the GPU; the SpMM is within 1e-5 of float64); under float16 autocast
|d| <= 2e-2 * scale, where scale is the largest magnitude of the reference
tensor."""
import copy

import numpy as np
import pytest
import scipy.sparse as sps
import torch

from graph_rws_amd import synth
from graph_rws_amd.data import BCSRGraph
from graph_rws_amd.helper import train_epoch_full
from graph_rws_amd.layers import BCSRGraphConv
from graph_rws_amd.models import GCN_BCSR

pytestmark = pytest.mark.gpu


def _dense(g):
    A = sps.csr_matrix((g.values.numpy().astype(np.float64), g.col_idx.numpy(), g.row_ptr.numpy()),
                       shape=(g.num_nodes, g.num_nodes))
    return torch.from_numpy(A.toarray())


def _close(a, b, tol):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    scale = max(float(b.abs().max()), 1e-30)
    d = float((a - b).abs().max())
    assert d <= tol * scale, f"max |diff| {d:.3e} > {tol:g} * {scale:.3e}"


@pytest.mark.parametrize("tc", [8, 16])
@pytest.mark.parametrize("fin,fout,xgrad", [(48, 24, True), (24, 48, True), (40, 24, False),
                                            (64, 24, False)])
def test_graphconv_forward_backward_f32(cuda_device, tc, fin, fout, xgrad):
    """Both associations of A X W: X-first (48->24 with dX, 64->24 without)
    and aggregate-first (24->48 with dX, 40->24 without)."""
    print(f"case graphconv f32 tc={tc} {fin}->{fout} xgrad={xgrad}", flush=True)
    torch.manual_seed(0)
    g = synth.chung_lu(1500, 20000, 2.2, seed=3)
    G = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes, tile_cols=tc,
                           device=cuda_device)
    conv = BCSRGraphConv(fin, fout).to(cuda_device)
    X = torch.randn(g.num_nodes, fin, device=cuda_device, requires_grad=xgrad)
    R = torch.randn(g.num_nodes, fout, device=cuda_device)
    # without features_target the self path is padded to the 16W output rows
    # (layer.py:159-166); with it the output is trimmed to the target rows
    assert conv(G, X).shape == (16 * G.num_windows, fout)
    out = conv(G, X, features_target=X)
    assert out.shape == (g.num_nodes, fout)
    (out * R).sum().backward()

    A = _dense(g)
    Xd = X.detach().double().cpu().requires_grad_(xgrad)
    Wn = conv.weight_neigh.detach().double().cpu().requires_grad_(True)
    Ws = conv.weight_self.detach().double().cpu().requires_grad_(True)
    ref = A @ (Xd @ Wn) + Xd @ Ws
    (ref * R.double().cpu()).sum().backward()
    _close(out, ref, 1e-4)
    if xgrad:
        _close(X.grad, Xd.grad, 1e-4)
    _close(conv.weight_neigh.grad, Wn.grad, 1e-4)
    _close(conv.weight_self.grad, Ws.grad, 1e-4)


def _reference_forward(model, A, X):
    """float64 dense restatement of GCN_BCSR.forward in eval mode."""
    h = X.double()
    L = len(model.layers)
    for l, layer in enumerate(model.layers):
        Wn = layer.weight_neigh.detach().double().cpu()
        Ws = layer.weight_self.detach().double().cpu()
        h = A @ (h @ Wn) + h @ Ws
        if l < L - 1:
            h = torch.relu(h)
            n = model.norms[l]
            h = torch.nn.functional.layer_norm(h, (h.shape[1],), n.weight.detach().double().cpu(),
                                               n.bias.detach().double().cpu(), n.eps)
    return h


def test_gcn_forward_matches_dense_reference(cuda_device):
    print("case gcn forward c1", flush=True)
    torch.manual_seed(1)
    g = synth.config_graph("c1")
    G = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes, tile_cols=16,
                           device=cuda_device)
    X = synth.features(g.num_nodes, 1433, kind="binary", seed=2, device=cuda_device)
    model = GCN_BCSR(1433, 16, 7, 2, dropout=0.5, use_checkpoint=False).to(cuda_device).eval()
    with torch.no_grad():
        out = model(G, X)
    ref = _reference_forward(model, _dense(g), X.cpu())
    _close(out, ref, 1e-4)
    # inference path (model.py:268-285): no target slicing, so like the
    # reference it returns the 16W padded rows; the first n equal forward's
    out2 = model.inference(G, X)
    assert out2.shape[0] == 16 * G.num_windows
    _close(out2[: g.num_nodes], ref, 1e-4)


def test_gcn_forward_f16_autocast(cuda_device):
    print("case gcn forward f16 autocast", flush=True)
    torch.manual_seed(2)
    g = synth.config_graph("c2", scale=0.05)
    G = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes, tile_cols=16,
                           device=cuda_device, values_dtype=torch.float16)
    X = synth.features(g.num_nodes, 128, seed=3, device=cuda_device).half()
    model = GCN_BCSR(128, 64, 10, 3, dropout=0.0, use_checkpoint=False).to(cuda_device).eval()
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
        out = model(G, X)
    A = _dense(g)
    A = A.to(torch.float16).double()  # the quantised values the device multiplies
    ref = _reference_forward(model, A, X.double().cpu())
    _close(out.float(), ref, 2e-2)


def test_gcn_training_step_matches_reference_grads(cuda_device):
    """One train_epoch_full step (engine.py:44-83): gradients of every
    parameter match float64 autograd through the dense restatement."""
    print("case gcn train step", flush=True)
    torch.manual_seed(3)
    g = synth.config_graph("c1")
    G = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes, tile_cols=8,
                           device=cuda_device)
    X = synth.features(g.num_nodes, 1433, kind="binary", seed=2, device=cuda_device)
    labels = torch.randint(0, 7, (g.num_nodes,), device=cuda_device)
    train_idx = torch.arange(0, g.num_nodes, 3, device=cuda_device)
    model = GCN_BCSR(1433, 16, 7, 2, dropout=0.0, use_checkpoint=False).to(cuda_device)
    ref_model = copy.deepcopy(model).cpu().double()

    opt = torch.optim.SGD(model.parameters(), lr=0.0)  # lr 0: keep params for the check
    loss, acc = train_epoch_full(model, G, X, labels, train_idx, opt, cuda_device)

    A = _dense(g)
    h = X.double().cpu()
    for l, layer in enumerate(ref_model.layers):
        h = A @ (h @ layer.weight_neigh) + h @ layer.weight_self
        if l < 1:
            h = ref_model.norms[l](torch.relu(h))
    ref_loss = torch.nn.functional.cross_entropy(h[train_idx.cpu()], labels.cpu()[train_idx.cpu()])
    ref_loss.backward()
    total = torch.sqrt(sum((p.grad ** 2).sum() for p in ref_model.parameters()))
    clip = min(1.0, 1.0 / (float(total) + 1e-6))
    rl = float(ref_loss.detach())
    assert abs(loss - rl) <= 1e-4 * abs(rl)
    for (n, p), (_, q) in zip(model.named_parameters(), ref_model.named_parameters()):
        _close(p.grad, q.grad * clip, 1e-3)


def test_gcn_loss_decreases(cuda_device):
    print("case gcn loss decreases", flush=True)
    torch.manual_seed(4)
    g = synth.config_graph("c1")
    G = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes, tile_cols=16,
                           device=cuda_device)
    X = synth.features(g.num_nodes, 1433, kind="binary", seed=2, device=cuda_device)
    labels = torch.randint(0, 7, (g.num_nodes,), device=cuda_device)
    idx = torch.arange(g.num_nodes, device=cuda_device)
    model = GCN_BCSR(1433, 16, 7, 2, dropout=0.5).to(cuda_device)
    opt = torch.optim.Adam(model.parameters(), lr=0.01)
    losses = [train_epoch_full(model, G, X, labels, idx, opt, cuda_device)[0] for _ in range(30)]
    assert losses[-1] < 0.8 * losses[0], losses


@pytest.mark.parametrize("dt", [None, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("fout", [16, 47, 256])
def test_fused_self_path_matches_separate_add(cuda_device, dt, fout):
    """The convolution's self product added in the SpMM epilogue (one GEMM
    for X W_n and X W_s) against the separate beta=1 GEMM: outputs within
    the rounding of the sum, and the same gradients (the backward is the
    same computation)."""
    from graph_rws_amd.layers import layer as layer_mod
    print(f"case fused-self dt={dt} fout={fout}", flush=True)
    g = synth.chung_lu(3000, 60000, 2.1, seed=fout)
    G = BCSRGraph.from_csr(g.row_ptr.to(cuda_device), g.col_idx.to(cuda_device), g.values.to(cuda_device),
                           g.num_nodes, g.num_nodes, tile_cols=16, device=cuda_device,
                           values_dtype=torch.float32 if dt is None else dt)
    torch.manual_seed(fout)
    conv = BCSRGraphConv(96, fout).to(cuda_device)
    X0 = synth.features(g.num_nodes, 96, seed=3, device=cuda_device)
    outs, grads = [], []
    for fused in (True, False):
        layer_mod.FUSED_SELF = fused
        try:
            X = X0.clone().requires_grad_(True)
            conv.zero_grad()
            with torch.autocast("cuda", dtype=dt or torch.float16, enabled=dt is not None):
                y = conv(G, X, features_target=X)           # the model's full-graph call
            y.float().square().sum().backward()
            outs.append(y.detach().float())
            grads.append([X.grad.clone(), conv.weight_neigh.grad.clone(), conv.weight_self.grad.clone()])
        finally:
            layer_mod.FUSED_SELF = True
    torch.cuda.synchronize()
    tol = 1e-5 if dt is None else 2e-2
    scale = float(outs[1].abs().max())
    assert float((outs[0] - outs[1]).abs().max()) <= tol * scale
    for a, b in zip(grads[0], grads[1]):
        assert float((a - b).abs().max()) <= tol * float(b.abs().max()) + 1e-6


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("xgrad", [False, True])
def test_aggregate_first_on_padded_width(cuda_device, dt, xgrad):
    """An aggregate-first layer (112 -> 256) whose input the graph gathers
    through a zero-padded 128-element copy runs its GEMMs over the padded
    width: same output (within the rounding of the GEMMs) and the same
    gradients as over the 112 columns, weight gradients of the weights'
    own shape."""
    from graph_rws_amd.layers import layer as layer_mod
    print(f"case padded-aggregate dt={dt} xgrad={xgrad}", flush=True)
    g = synth.chung_lu(3000, 200000, 2.1, seed=21)
    G = BCSRGraph.from_csr(g.row_ptr.to(cuda_device), g.col_idx.to(cuda_device), g.values.to(cuda_device),
                           g.num_nodes, g.num_nodes, tile_cols=16, device=cuda_device, values_dtype=dt)
    assert G.num_tiles * 16 >= 8 * g.num_nodes                  # the graph gathers through a copy
    torch.manual_seed(5)
    conv = BCSRGraphConv(112, 256).to(cuda_device)
    X0 = synth.features(g.num_nodes, 112, seed=4, device=cuda_device).to(dt)
    assert G.padded_input(X0) is not None and G.padded_input(X0).shape[1] == 128
    outs, grads = [], []
    for pad in (True, False):
        layer_mod.PAD_AGGREGATE = pad
        try:
            X = X0.clone().requires_grad_(xgrad)
            conv.zero_grad()
            with torch.autocast("cuda", dtype=dt):
                y = conv(G, X, features_target=X)
            y.float().square().sum().backward()
            outs.append(y.detach().float())
            grads.append([conv.weight_neigh.grad.clone(), conv.weight_self.grad.clone()]
                         + ([X.grad.clone()] if xgrad else []))
        finally:
            layer_mod.PAD_AGGREGATE = True
    torch.cuda.synchronize()
    assert float((outs[0] - outs[1]).abs().max()) <= 2e-2 * float(outs[1].abs().max())
    for a, b in zip(grads[0], grads[1]):
        assert a.shape == b.shape
        assert float((a - b).abs().max()) <= 2e-2 * float(b.abs().max()) + 1e-6
